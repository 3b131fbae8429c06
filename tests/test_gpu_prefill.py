"""GPU parity of chunked prefill (bmo_kv_ring_prefill) against the float64
oracle orc_ring_prefill_f64: outputs within |gpu - ref| <= 2e-3 + 1e-3 |ref|,
and the ring bit-exact after the chunk is committed.

Inputs are bf16: seeded normals rounded to bf16 on the
host, handed to the GPU as bfloat16 and to the oracle as the same values in
fp32.  The oracle quantizes the chunk's K/V with its Q4_0 restatement, so the
committed blocks must match byte for byte."""
import numpy as np
import pytest

import oracle
from _ringsim import Mirror, check_close

pytestmark = pytest.mark.gpu


def _i32(torch, vals):
    return torch.tensor(list(vals), dtype=torch.int32, device="cuda")


def _bf16_normals(seed, shape):
    return oracle.round_bf16(oracle.normal(seed, int(np.prod(shape)))).reshape(shape)


def _run(gpu, m, layer, entries, n_tok, n_heads, seed, session_ids=None):
    """entries: list of (session or None for a skipped entry, pos0)."""
    n_batch = len(entries)
    d, n_kv = m.d, m.n_kv
    q = _bf16_normals(seed, (n_batch, n_tok, n_heads, d))
    k = _bf16_normals(seed + 1, (n_batch, n_tok, n_kv, d))
    v = _bf16_normals(seed + 2, (n_batch, n_tok, n_kv, d))
    out = gpu.full((n_batch, n_tok, n_heads, d), float("nan"), dtype=gpu.float32, device="cuda")
    pos0 = [p for _, p in entries]
    sids = session_ids if session_ids is not None else None
    m.ring.prefill(layer, _i32(gpu, pos0), m.dev(q, gpu.bfloat16), m.dev(k, gpu.bfloat16),
                   m.dev(v, gpu.bfloat16), out, n_heads, n_tok=n_tok,
                   session_ids=None if sids is None else _i32(gpu, sids), stream=m.stream)
    gpu.cuda.synchronize()
    got = out.cpu().numpy()
    for b, (s, p0) in enumerate(entries):
        if s is None:
            assert np.all(got[b] == 0.0), f"skipped entry {b} must be zeroed"
            continue
        kc, vc = m.orc[(layer, s)]
        ref = oracle.ring_prefill_f64(kc, vc, p0, q[b], k[b], v[b], n_heads)
        check_close(got[b], ref, f"prefill entry {b} pos0={p0}")
        m.assert_ring_equal(layer, s)


@pytest.mark.parametrize("pos0,n_tok", [
    (1000, 256),   # BASELINE config 5, ring history full (reduced to 4 heads)
    (0, 256),      # config 5, first chunk: empty history
    (500, 100),    # chunk wraps the ring end, partial query tile
    (700, 37),
    (3, 1),        # one token: the decode case
    (512, 512),    # chunk as long as the ring
])
def test_prefill_parity(gpu, pos0, n_tok):
    n_heads, d, n_ctx = 4, 128, 512
    m = Mirror(gpu, 2, 1, n_heads, d, n_ctx)
    layer = 1
    m.fill_range(layer, 0, 0, pos0, seed=9000 + pos0)
    _run(gpu, m, layer, [(0, pos0)], n_tok, n_heads, seed=100 + n_tok)


@pytest.mark.parametrize("n_ctx,pos0,n_tok,n_heads,n_kv", [
    (40, 90, 30, 4, 4),     # 32-key ring tiles wrap inside the ring (staged path)
    (8, 5, 8, 4, 4),        # an 8-slot ring (the depformer's), chunk as long as the ring
    (72, 100, 60, 8, 2),    # staged chunk (4 query heads per kv head)
    (100, 1000, 100, 4, 4),
    (96, 70, 9, 4, 4),      # ring tiles aligned, last one partial
    (1024, 3000, 256, 2, 2),   # a 1024-slot ring: 33 ring tiles, several loop passes
    (1024, 3001, 200, 2, 2),   # the same with the chunk start off the 32-slot grid
])
def test_prefill_ring_sizes(gpu, n_ctx, pos0, n_tok, n_heads, n_kv):
    m = Mirror(gpu, 1, 1, n_kv, 128, n_ctx)
    m.fill_range(0, 0, 0, pos0, seed=300 + n_ctx)
    _run(gpu, m, 0, [(0, pos0)], n_tok, n_heads, seed=310 + n_ctx)


@pytest.mark.parametrize("n_ctx,pos0,n_tok,n_heads,n_kv", [
    (64, 200, 64, 4, 4),    # direct path, ring a multiple of 32 (16 waves x 16 queries)
    (512, 700, 256, 2, 2),  # the same at the temporal ring's size, a full chunk
    (64, 90, 40, 8, 2),     # staged path (4 query heads per kv head), aligned ring
    (40, 90, 30, 4, 2),     # staged path, ring not a multiple of 32
])
def test_prefill_head_dim_64(gpu, n_ctx, pos0, n_tok, n_heads, n_kv):
    m = Mirror(gpu, 1, 1, n_kv, 64, n_ctx)
    m.fill_range(0, 0, 0, pos0, seed=400 + n_ctx)
    _run(gpu, m, 0, [(0, pos0)], n_tok, n_heads, seed=410 + n_tok)


def test_prefill_gqa_and_head_dim_64(gpu):
    m = Mirror(gpu, 1, 1, 2, 128, 96)
    m.fill_range(0, 0, 0, 150, seed=31)
    _run(gpu, m, 0, [(0, 150)], 70, 8, seed=32)      # 4 query heads per kv head
    m2 = Mirror(gpu, 1, 1, 4, 64, 40)
    m2.fill_range(0, 0, 0, 55, seed=33)
    _run(gpu, m2, 0, [(0, 55)], 20, 4, seed=34)      # depformer head size


def test_prefill_batched_sessions_and_skips(gpu):
    n_kv, d, n_ctx = 2, 128, 128
    m = Mirror(gpu, 1, 4, n_kv, d, n_ctx)
    hist = {0: 300, 2: 0, 3: 130}
    for s, p in hist.items():
        m.fill_range(0, s, 0, p, seed=40 + s)
    before = (m.ring.export_q4_0(0, 1, 0, 0, n_ctx), m.ring.export_q4_0(0, 1, 1, 0, n_ctx))
    # entry 1 names session 7 (out of range) -> skipped
    entries = [(3, 130), (None, 5), (0, 300), (2, 0)]
    _run(gpu, m, 0, entries, 48, n_kv, seed=50, session_ids=[3, 7, 0, 2])
    assert np.array_equal(m.ring.export_q4_0(0, 1, 0, 0, n_ctx), before[0])
    assert np.array_equal(m.ring.export_q4_0(0, 1, 1, 0, n_ctx), before[1])


def test_prefill_then_decode_continues(gpu):
    """Chunks then single-token steps on one session: the ring state after
    prefill is exactly what decode reads next."""
    n_heads, d, n_ctx = 4, 128, 64
    m = Mirror(gpu, 1, 1, n_heads, d, n_ctx)
    _run(gpu, m, 0, [(0, 0)], 40, n_heads, seed=60)
    _run(gpu, m, 0, [(0, 40)], 40, n_heads, seed=61)   # wraps, overwrites the first chunk
    out = gpu.full((n_heads * d,), float("nan"), dtype=gpu.float32, device="cuda")
    for p in range(80, 84):
        q = oracle.normal(70 + p, n_heads * d)
        k = oracle.normal(80 + p, n_heads * d)
        v = oracle.normal(90 + p, n_heads * d)
        m.ring.append_decode(0, _i32(gpu, [p]), m.dev(q), m.dev(k), m.dev(v), out, n_heads,
                             stream=m.stream)
        m.oracle_append(0, 0, p, k, v)
        gpu.cuda.synchronize()
        check_close(out.cpu().numpy().reshape(n_heads, d), m.oracle_decode(0, 0, p, q, n_heads),
                    f"decode after prefill, pos {p}")
    m.assert_ring_equal(0, 0)


def test_prefill_argument_errors(gpu):
    from bmo_jetson_amd import KVRing, RingError
    ring = KVRing(1, 2, 2, 128, 16)
    x = gpu.zeros(2 * 17 * 2 * 128, dtype=gpu.bfloat16, device="cuda")
    out = gpu.zeros(2 * 17 * 2 * 128, dtype=gpu.float32, device="cuda")
    pos = _i32(gpu, [0, 0])
    with pytest.raises(RingError) as e:
        ring.prefill(0, pos, x, x, x, out, 2, n_tok=17)     # longer than the ring
    assert e.value.rc == 2
    with pytest.raises(RingError) as e:
        ring.prefill(1, pos, x, x, x, out, 2, n_tok=4)      # bad layer
    assert e.value.rc == 2
    with pytest.raises(RingError) as e:
        ring.prefill(0, pos, x, x, x, out, 3, n_tok=4)      # heads not a multiple of kv heads
    assert e.value.rc == 2
    ring.prefill(0, pos, x, x, x, out, 2, n_tok=4)
    gpu.cuda.synchronize()
    assert ring.last_error() is None
    ring.close()


def test_prefill_query_range(gpu):
    """Large query elements stay within the usual bar: each query row enters
    the matrix cores scaled by its own power of two, so no fixed fp16 range
    applies (4e5, 1e6 and 1e12 in three rows; a single fp16 scaling of
    q * scale * log2(e) would overflow past about 5.1e5)."""
    n_heads, d, n_ctx, pos0, n_tok = 2, 128, 64, 100, 16
    m = Mirror(gpu, 1, 1, n_heads, d, n_ctx)
    m.fill_range(0, 0, 0, pos0, seed=77)
    q = _bf16_normals(78, (1, n_tok, n_heads, d))
    k = _bf16_normals(79, (1, n_tok, n_heads, d))
    v = _bf16_normals(80, (1, n_tok, n_heads, d))
    q[0, 3, 0, 5] = 4.0e5
    q[0, 9, 1, 17] = 1.0e6
    q[0, 12, 0, 100] = 1.0e12
    q = oracle.round_bf16(q)
    out = gpu.full((1, n_tok, n_heads, d), float("nan"), dtype=gpu.float32, device="cuda")
    m.ring.prefill(0, _i32(gpu, [pos0]), m.dev(q, gpu.bfloat16), m.dev(k, gpu.bfloat16),
                   m.dev(v, gpu.bfloat16), out, n_heads, n_tok=n_tok, stream=m.stream)
    gpu.cuda.synchronize()
    got = out.cpu().numpy()[0]
    kc, vc = m.orc[(0, 0)]
    ref = oracle.ring_prefill_f64(kc, vc, pos0, q[0], k[0], v[0], n_heads)
    check_close(got, ref, "large query elements")
    m.assert_ring_equal(0, 0)   # (the oracle's prefill appended the chunk)
