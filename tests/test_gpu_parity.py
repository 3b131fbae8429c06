"""GPU parity: the HIP kernels (called through the C ABI) against the CPU
oracle on the same seeded inputs.

  * append / write: bit-exact Q4_0 blocks (scale bits and code bytes);
  * decode / fused append+decode / node launcher: within
    |gpu - ref| <= 2e-3 + 1e-3 |ref| of the float64 oracle, and the ring
    state after a fused call bit-exact.
"""
import json
import os

import numpy as np
import pytest

import oracle
from _ringsim import Mirror, check_close
from bmo_jetson_amd import KVRing, launch_decode_attention, stripe_bytes

pytestmark = pytest.mark.gpu

KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "q4_0_kat.json")))


def _i32(torch, vals):
    return torch.tensor(list(vals), dtype=torch.int32, device="cuda")


def _adversarial_rows(n_rows, width, seed):
    """Rows mixing the blocks most likely to expose a quantizer slip."""
    rng = np.random.default_rng(seed)
    nb = n_rows * width // 32
    blocks = oracle.normal(seed, nb * 32).reshape(nb, 32)
    kind = np.arange(nb) % 12
    for i in range(nb):
        x = blocks[i]
        k = kind[i]
        if k == 1:
            x *= np.where(rng.random(32) < 0.05, 8.0, 1.0).astype(np.float32)
        elif k == 2:
            x[:] = 0.0
        elif k == 3:
            x[:] = -0.0
        elif k == 4:
            x[rng.integers(32)] = -np.abs(x).max() - 1.0
            x[rng.integers(32)] = np.abs(x).max()  # magnitude tie, later index
        elif k == 5:
            x *= np.float32(2.0 ** rng.integers(-140, -120))  # subnormal / tiny scales
        elif k == 6:
            x *= np.float32(2.0 ** rng.integers(14, 20))       # fp16 overflowing scales
        elif k == 7:
            x[:] = np.round(x * 2) / 2                         # exact halves
        elif k == 8:
            x[:] = (np.arange(32) - 16).astype(np.float32) * np.float32(rng.random() + 0.1)
        elif k == 9:
            x[:] = np.float32(rng.random() + 0.5) * np.sign(x)  # constant magnitude
        elif k == 10:
            x *= np.float32(2.0 ** rng.integers(-30, -14))     # fp16-subnormal scales
        elif k == 11:
            # non-finite values take the quantizer's literal path: a NaN is
            # never the max and codes as 0; an infinity gives an infinite d
            sel = rng.integers(4)
            x[rng.integers(32)] = (np.nan, np.inf, -np.inf, np.nan)[sel]
            if sel == 3:
                x *= np.float32(2.0 ** -123)                   # with a near-boundary scale
    return blocks.reshape(n_rows, width)


@pytest.mark.parametrize("d", [128, 64])
def test_write_bit_exact_kats(gpu, d):
    cases = [np.array(c["x"], np.float32) for c in KAT["cases"]]
    nblk = d // 32
    n_kv = 2
    rows = []
    for r in range(0, len(cases), nblk * n_kv):
        blocks = [cases[(r + i) % len(cases)] for i in range(nblk * n_kv)]
        rows.append(np.concatenate(blocks).reshape(n_kv, d))
    k = np.stack(rows)
    v = -k[::-1].copy()
    m = Mirror(gpu, 1, 1, n_kv, d, 16)
    m.write(0, 0, 0, k, v)
    gpu.cuda.synchronize()
    m.assert_ring_equal(0, 0)


@pytest.mark.parametrize("d,n_ctx", [(128, 512), (64, 8)])
def test_write_bit_exact_adversarial(gpu, d, n_ctx):
    n_kv = 4
    m = Mirror(gpu, 2, 2, n_kv, d, n_ctx)
    for layer in range(2):
        for s in range(2):
            n = n_ctx
            k = _adversarial_rows(n * n_kv, d, 100 + layer * 10 + s).reshape(n, n_kv, d)
            v = _adversarial_rows(n * n_kv, d, 200 + layer * 10 + s).reshape(n, n_kv, d)
            m.write(layer, s, 1000 * s + layer, k, v)
    gpu.cuda.synchronize()
    for layer in range(2):
        for s in range(2):
            m.assert_ring_equal(layer, s)


def test_append_batched_bit_exact(gpu):
    n_sess, n_kv, d, n_ctx = 6, 8, 128, 32
    m = Mirror(gpu, 1, n_sess, n_kv, d, n_ctx)
    pos = [0, 31, 32, 77, 1000, 5]
    sids = [3, 0, 5, 1, 4, 2]
    k = _adversarial_rows(n_sess * n_kv, d, 7).reshape(n_sess, n_kv, d)
    v = _adversarial_rows(n_sess * n_kv, d, 8).reshape(n_sess, n_kv, d)
    m.ring.append(0, _i32(gpu, pos), m.dev(k), m.dev(v), session_ids=_i32(gpu, sids),
                  stream=m.stream)
    for b in range(n_sess):
        m.oracle_append(0, sids[b], pos[b], k[b], v[b])
    gpu.cuda.synchronize()
    for s in range(n_sess):
        m.assert_ring_equal(0, s)


DECODE_CASES = [
    # (n_heads, n_kv, d, n_ctx, pos)       config
    (32, 32, 128, 512, 700),   # W=512, write head at 700 (slot 188)
    (32, 32, 128, 512, 0),     # window of one key
    (32, 32, 128, 512, 1),
    (32, 32, 128, 512, 37),    # partial window
    (32, 32, 128, 512, 510),
    (32, 32, 128, 512, 511),   # ring exactly full
    (32, 32, 128, 512, 512),   # first wrap
    (32, 32, 128, 512, 4095),
    (16, 16, 64, 8, 0),        # depformer, steps 1..8
    (16, 16, 64, 8, 3),
    (16, 16, 64, 8, 7),
    (8, 2, 128, 64, 100),      # GQA
    (4, 4, 128, 1000, 2500),   # n_ctx not a power of two
    (4, 4, 64, 3, 10),         # tiny ring
]


@pytest.mark.parametrize("n_heads,n_kv,d,n_ctx,pos", DECODE_CASES)
def test_decode_parity(gpu, n_heads, n_kv, d, n_ctx, pos):
    m = Mirror(gpu, 2, 1, n_kv, d, n_ctx)
    layer = 1
    m.fill_range(layer, 0, 0, pos + 1, seed=0xB0A00001 + pos)  # whole window ending at pos
    q = oracle.normal(0xB0A00001 ^ pos, n_heads * d)
    out = gpu.full((n_heads * d,), float("nan"), dtype=gpu.float32, device="cuda")
    m.ring.decode(layer, _i32(gpu, [pos]), m.dev(q), out, n_heads, stream=m.stream)
    gpu.cuda.synchronize()
    ref = m.oracle_decode(layer, 0, pos, q, n_heads)
    check_close(out.cpu().numpy().reshape(n_heads, d), ref, f"decode pos={pos}")


@pytest.mark.parametrize("n_heads,n_kv,d,n_ctx,pos", DECODE_CASES)
def test_fused_append_decode_parity(gpu, n_heads, n_kv, d, n_ctx, pos):
    m = Mirror(gpu, 2, 1, n_kv, d, n_ctx)
    layer = 0
    m.fill_range(layer, 0, 0, pos, seed=0xB0A00004 + pos)  # window before the new token
    q = oracle.normal(11 + pos, n_heads * d)
    k = oracle.normal(12 + pos, n_kv * d)
    v = oracle.normal(13 + pos, n_kv * d)
    out = gpu.full((n_heads * d,), float("nan"), dtype=gpu.float32, device="cuda")
    m.ring.append_decode(layer, _i32(gpu, [pos]), m.dev(q), m.dev(k), m.dev(v), out, n_heads,
                         stream=m.stream)
    m.oracle_append(layer, 0, pos, k, v)
    gpu.cuda.synchronize()
    ref = m.oracle_decode(layer, 0, pos, q, n_heads)
    check_close(out.cpu().numpy().reshape(n_heads, d), ref, f"fused pos={pos}")
    m.assert_ring_equal(layer, 0)


@pytest.mark.parametrize("d,n_ctx,theta", [(128, 48, None), (64, 8, None), (128, 48, 10000.0),
                                           (64, 8, 500000.0)])
def test_fused_append_adversarial_bit_exact(gpu, d, n_ctx, theta):
    """The fused call quantizes the current token's rows with the wave spread
    over the blocks (BL lanes per block); its ring writes must match the
    oracle quantizer bit for bit on the adversarial blocks (ties of +max and
    -max, NaN, infinities, zero and -0 blocks, subnormal and fp16-overflowing
    scales), with and without RoPE, GQA, one entry per session."""
    n_sess, n_kv, n_heads = 6, 4, 8
    m = Mirror(gpu, 1, n_sess, n_kv, d, n_ctx)
    sids = [4, 0, 5, 2, 1, 3]
    for step in range(3):
        pos = [(7 * b + 3 * step) % 50 + step for b in range(n_sess)]
        k = _adversarial_rows(n_sess * n_kv, d, 300 + step).reshape(n_sess, n_kv, d)
        v = _adversarial_rows(n_sess * n_kv, d, 400 + step).reshape(n_sess, n_kv, d)
        q = oracle.normal(500 + step, n_sess * n_heads * d)
        out = gpu.empty((n_sess * n_heads * d,), dtype=gpu.float32, device="cuda")
        m.ring.append_decode(0, _i32(gpu, pos), m.dev(q), m.dev(k), m.dev(v), out, n_heads,
                             session_ids=_i32(gpu, sids), stream=m.stream, rope_theta=theta)
        for b in range(n_sess):
            kb = k[b] if theta is None else oracle.rope_interleaved(k[b], pos[b], theta)
            m.oracle_append(0, sids[b], pos[b], kb, v[b])
        gpu.cuda.synchronize()
        for s in range(n_sess):
            m.assert_ring_equal(0, s)


def test_batched_sessions_ids_and_invalid_entries(gpu):
    n_sess, n_heads, d, n_ctx = 7, 8, 128, 96
    m = Mirror(gpu, 1, n_sess, n_heads, d, n_ctx)
    pos = [5, 95, 96, 300, 0, -1, 12]
    sids = [6, 0, 2, 3, 1, 4, 9]  # entry 5 has pos -1, entry 6 a bad session id
    for b, (s, p) in enumerate(zip(sids, pos)):
        if 0 <= s < n_sess and p >= 0:
            m.fill_range(0, s, 0, p, seed=300 + b)
    before = {s: (m.ring.export_q4_0(0, s, 0, 0, n_ctx), m.ring.export_q4_0(0, s, 1, 0, n_ctx))
              for s in (4, 5)}
    q = oracle.normal(21, n_sess * n_heads * d).reshape(n_sess, n_heads, d)
    k = oracle.normal(22, n_sess * n_heads * d).reshape(n_sess, n_heads, d)
    v = oracle.normal(23, n_sess * n_heads * d).reshape(n_sess, n_heads, d)
    out = gpu.full((n_sess, n_heads, d), 7.0, dtype=gpu.float32, device="cuda")
    m.ring.append_decode(0, _i32(gpu, pos), m.dev(q), m.dev(k), m.dev(v), out, n_heads,
                         session_ids=_i32(gpu, sids), stream=m.stream)
    gpu.cuda.synchronize()
    got = out.cpu().numpy()
    for b, (s, p) in enumerate(zip(sids, pos)):
        if 0 <= s < n_sess and p >= 0:
            m.oracle_append(0, s, p, k[b], v[b])
            check_close(got[b], m.oracle_decode(0, s, p, q[b], n_heads), f"entry {b}")
            m.assert_ring_equal(0, s)
        else:
            assert np.all(got[b] == 0.0), f"skipped entry {b} must be zeroed"
    for s in (4, 5):  # untouched sessions keep their bytes
        assert np.array_equal(m.ring.export_q4_0(0, s, 0, 0, n_ctx), before[s][0])
        assert np.array_equal(m.ring.export_q4_0(0, s, 1, 0, n_ctx), before[s][1])


def test_sequence_of_steps_with_wrap(gpu):
    """Autoregressive use: fused steps p = 0 .. 2*n_ctx+3 on one session, each
    checked, so every slot is overwritten at least twice."""
    n_heads, d, n_ctx = 4, 64, 16
    m = Mirror(gpu, 1, 1, n_heads, d, n_ctx)
    out = gpu.full((n_heads * d,), float("nan"), dtype=gpu.float32, device="cuda")
    for p in range(2 * n_ctx + 4):
        q = oracle.normal(1000 + p, n_heads * d)
        k = oracle.normal(2000 + p, n_heads * d)
        v = oracle.normal(3000 + p, n_heads * d)
        m.ring.append_decode(0, _i32(gpu, [p]), m.dev(q), m.dev(k), m.dev(v), out, n_heads,
                             stream=m.stream)
        m.oracle_append(0, 0, p, k, v)
        gpu.cuda.synchronize()
        check_close(out.cpu().numpy().reshape(n_heads, d), m.oracle_decode(0, 0, p, q, n_heads),
                    f"step {p}")
    m.assert_ring_equal(0, 0)


@pytest.mark.parametrize("use_pos_dev", [False, True])
@pytest.mark.parametrize("n_heads,n_kv,d,n_ctx,pos", [(32, 32, 128, 512, 700), (16, 16, 64, 8, 5),
                                                      (8, 4, 128, 32, 40)])
def test_node_launcher(gpu, use_pos_dev, n_heads, n_kv, d, n_ctx, pos):
    """bmo_launch_decode_attention over a ring allocated as the reference
    allocates its cache (n_heads head slots, one session)."""
    n_layers, layer = 3, 2
    m = Mirror(gpu, n_layers, 1, n_heads, d, n_ctx)
    # history for the n_kv live heads; the reference leaves slots >= n_kv unused
    lo = max(0, pos - n_ctx + 1)
    n = pos - lo
    if n:
        kh = np.zeros((n, n_heads, d), np.float32)
        vh = np.zeros((n, n_heads, d), np.float32)
        kh[:, :n_kv] = oracle.normal(41, n * n_kv * d).reshape(n, n_kv, d)
        vh[:, :n_kv] = oracle.normal(42, n * n_kv * d).reshape(n, n_kv, d)
        m.write(layer, 0, lo, kh, vh)
    q = oracle.normal(43, n_heads * d)
    k = oracle.normal(44, n_kv * d)
    v = oracle.normal(45, n_kv * d)
    out = gpu.full((n_heads * d,), float("nan"), dtype=gpu.float32, device="cuda")
    pos_dev = _i32(gpu, [pos]) if use_pos_dev else None
    launch_decode_attention(m.dev(q), m.dev(k), m.dev(v), m.ring.k_base, m.ring.v_base, out, d,
                            n_heads, n_kv, n_ctx, 0 if use_pos_dev else pos, layer,
                            stream=m.stream, pos_dev=pos_dev)
    gpu.cuda.synchronize()
    kc, vc = m.orc[(layer, 0)]
    kfull = np.zeros((n_heads, d), np.float32)
    vfull = np.zeros((n_heads, d), np.float32)
    kfull[:n_kv] = k.reshape(n_kv, d)
    vfull[:n_kv] = v.reshape(n_kv, d)
    # the kernel writes kv heads 0..n_kv-1 only; mirror that
    kq, vq = kc[:n_kv].copy(), vc[:n_kv].copy()
    oracle.ring_append(kq, vq, pos, kfull[:n_kv], vfull[:n_kv])
    ref = oracle.ring_decode_f64(kq, vq, pos, q, n_heads)
    check_close(out.cpu().numpy().reshape(n_heads, d), ref, "node launcher")
    kc[:n_kv], vc[:n_kv] = kq, vq
    m.assert_ring_equal(layer, 0)


def test_copy_k_cache_f32_and_codes(gpu):
    n_kv, d, n_ctx = 4, 128, 40
    m = Mirror(gpu, 2, 3, n_kv, d, n_ctx)
    m.fill_range(1, 2, 0, 60, seed=51)
    gpu.cuda.synchronize()
    got = m.ring.get_k_cache_f32(1, 5, 30, session=2)
    ref = oracle.ring_copy_k_f32(m.orc[(1, 2)][0], 5, 30)
    assert np.array_equal(got, ref)
    buf = np.zeros(10, np.float32)
    assert m.ring.copy_k_cache_f32(1, 0, 1, buf, session=2) == -2         # too small
    big = np.zeros(n_ctx * n_kv * d + 1, np.float32)
    assert m.ring.copy_k_cache_f32(1, 30, 11, big, session=2) == -3       # slots past n_ctx
    assert m.ring.copy_k_cache_f32(2, 0, 1, big, session=2) == -3         # bad layer
    assert m.ring.copy_k_cache_f32(1, -1, 1, big, session=2) == -3
    assert m.ring.copy_k_cache_f32(1, 0, 0, big, session=2) == -1         # n_positions <= 0
    assert m.ring.copy_k_cache_f32(1, 0, 1, big, session=3) == -1         # bad session


def test_reset_and_import_export(gpu):
    n_kv, d, n_ctx = 2, 64, 8
    m = Mirror(gpu, 2, 3, n_kv, d, n_ctx)
    for s in range(3):
        for layer in range(2):
            m.fill_range(layer, s, 0, 9, seed=61 + s + 10 * layer)
    gpu.cuda.synchronize()
    snap = m.ring.export_q4_0(1, 1, 0, 0, n_ctx)
    m.ring.reset(1, stream=m.stream)
    gpu.cuda.synchronize()
    for layer in range(2):
        assert not m.ring.export_q4_0(layer, 1, 0, 0, n_ctx).any()
        assert not m.ring.export_q4_0(layer, 1, 1, 0, n_ctx).any()
        m.assert_ring_equal(layer, 0)
        m.assert_ring_equal(layer, 2)
    # a zeroed ring attends to zeros
    out = gpu.empty(n_kv * d, dtype=gpu.float32, device="cuda")
    m.ring.decode(0, _i32(gpu, [1, 5]), m.dev(oracle.normal(1, 2 * n_kv * d)), out, n_kv,
                  n_batch=1, session_ids=_i32(gpu, [1]), stream=m.stream)
    gpu.cuda.synchronize()
    assert np.all(out.cpu().numpy() == 0.0)
    m.ring.import_q4_0(1, 1, 0, 0, snap)
    assert np.array_equal(m.ring.export_q4_0(1, 1, 0, 0, n_ctx), snap)
    m.ring.reset(-1, stream=m.stream)
    gpu.cuda.synchronize()
    for s in range(3):
        assert not m.ring.export_q4_0(0, s, 1, 0, n_ctx).any()


def test_api_errors_on_device(gpu):
    from bmo_jetson_amd import RingError
    ring = KVRing(2, 2, 4, 128, 16)
    pos = _i32(gpu, [0, 0])
    x = gpu.zeros(2 * 4 * 128, dtype=gpu.float32, device="cuda")
    with pytest.raises(RingError) as e:
        ring.decode(2, pos, x, x, 4)
    assert e.value.rc == 2 and "layer" in ring.last_error()
    with pytest.raises(RingError) as e:
        ring.decode(0, pos, x, x, 6)  # not a multiple of n_kv_heads
    assert e.value.rc == 2
    with pytest.raises(RingError) as e:
        ring.append(0, pos, x, x, n_batch=3)
    assert e.value.rc == 2
    with pytest.raises(RingError) as e:
        ring.write(0, 0, 0, x, x, n_tok=17)
    assert e.value.rc == 2
    with pytest.raises(RingError) as e:
        ring.reset(5)
    assert e.value.rc == 2
    ring.decode(0, pos, x, x, 4)  # a good call clears the message
    assert ring.last_error() is None
    assert ring.geometry() == (2, 2, 4, 128, 16)
    assert ring.nbytes == (2 * 2 * 4) * stripe_bytes(128, 16)


# every (waves per unit, prefetch depth) shape compiled into launch_shape()
# (decode.hip)
SHAPES = ["1,1", "1,2", "1,3", "2,1", "4,1", "8,1", "8,2", "16,1"]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("d,n_ctx,pos", [(128, 512, 700), (128, 512, 130), (64, 8, 5), (64, 200, 450)])
@pytest.mark.parametrize("fused", [False, True])
def test_every_workgroup_shape(gpu, monkeypatch, shape, d, n_ctx, pos, fused):
    """Each compiled workgroup shape (waves per unit, prefetch depth), forced
    through BMO_ATTN_SHAPE, against the oracle."""
    monkeypatch.setenv("BMO_ATTN_SHAPE", shape)
    n_sess, n_heads, n_kv = 3, 8, 4
    m = Mirror(gpu, 1, n_sess, n_kv, d, n_ctx)
    # output buffers start as NaN so an element the kernel never writes fails
    poss = [pos, max(0, pos - 3), pos + 17]
    for s, p in enumerate(poss):
        m.fill_range(0, s, 0, p + (0 if fused else 1), seed=500 + s)
    q = oracle.normal(31, n_sess * n_heads * d).reshape(n_sess, n_heads, d)
    out = gpu.full((n_sess, n_heads, d), float("nan"), dtype=gpu.float32, device="cuda")
    if fused:
        k = oracle.normal(32, n_sess * n_kv * d).reshape(n_sess, n_kv, d)
        v = oracle.normal(33, n_sess * n_kv * d).reshape(n_sess, n_kv, d)
        m.ring.append_decode(0, _i32(gpu, poss), m.dev(q), m.dev(k), m.dev(v), out, n_heads,
                             stream=m.stream)
        for s, p in enumerate(poss):
            m.oracle_append(0, s, p, k[s], v[s])
    else:
        m.ring.decode(0, _i32(gpu, poss), m.dev(q), out, n_heads, stream=m.stream)
    gpu.cuda.synchronize()
    got = out.cpu().numpy()
    for s, p in enumerate(poss):
        check_close(got[s], m.oracle_decode(0, s, p, q[s], n_heads), f"shape {shape} entry {s}")
    if fused:
        for s in range(n_sess):
            m.assert_ring_equal(0, s)


@pytest.mark.parametrize("fused", [False, True])
def test_large_batch_default_shape(gpu, fused):
    """>= 512 (entry, head) units selects the batch shape (one wave per unit):
    64 sessions x 8 heads, random wrap points."""
    n_sess, n_heads, d, n_ctx = 64, 8, 128, 128
    m = Mirror(gpu, 2, n_sess, n_heads, d, n_ctx)
    rng = np.random.default_rng(5)
    poss = [int(x) for x in rng.integers(0, 3 * n_ctx, size=n_sess)]
    layer = 1
    for s, p in enumerate(poss):
        m.fill_range(layer, s, 0, p + (0 if fused else 1), seed=700 + s)
    q = oracle.normal(41, n_sess * n_heads * d).reshape(n_sess, n_heads, d)
    out = gpu.full((n_sess, n_heads, d), float("nan"), dtype=gpu.float32, device="cuda")
    if fused:
        k = oracle.normal(42, n_sess * n_heads * d).reshape(n_sess, n_heads, d)
        v = oracle.normal(43, n_sess * n_heads * d).reshape(n_sess, n_heads, d)
        m.ring.append_decode(layer, _i32(gpu, poss), m.dev(q), m.dev(k), m.dev(v), out, n_heads,
                             stream=m.stream)
        for s, p in enumerate(poss):
            m.oracle_append(layer, s, p, k[s], v[s])
    else:
        m.ring.decode(layer, _i32(gpu, poss), m.dev(q), out, n_heads, stream=m.stream)
    gpu.cuda.synchronize()
    got = out.cpu().numpy()
    worst = 0.0
    for s, p in enumerate(poss):
        mx, _ = check_close(got[s], m.oracle_decode(layer, s, p, q[s], n_heads), f"session {s}")
        worst = max(worst, mx)
    if fused:
        for s in range(0, n_sess, 7):
            m.assert_ring_equal(layer, s)


def test_b1_repeated_calls(gpu):
    """B=1 calls (16 waves per head merging in LDS): a run of calls at
    changing positions (full windows, wraps, fused and plain) on one ring."""
    n_heads, d, n_ctx = 32, 128, 512
    m = Mirror(gpu, 1, 1, n_heads, d, n_ctx)
    m.fill_range(0, 0, 0, 600, seed=77)
    out = gpu.full((n_heads * d,), float("nan"), dtype=gpu.float32, device="cuda")
    p = 600
    for step in range(6):
        q = oracle.normal(800 + step, n_heads * d)
        if step % 2:
            k = oracle.normal(900 + step, n_heads * d)
            v = oracle.normal(950 + step, n_heads * d)
            m.ring.append_decode(0, _i32(gpu, [p]), m.dev(q), m.dev(k), m.dev(v), out, n_heads,
                                 stream=m.stream)
            m.oracle_append(0, 0, p, k, v)
        else:
            m.ring.decode(0, _i32(gpu, [p - 1]), m.dev(q), out, n_heads, stream=m.stream)
        gpu.cuda.synchronize()
        ref = m.oracle_decode(0, 0, p if step % 2 else p - 1, q, n_heads)
        check_close(out.cpu().numpy().reshape(n_heads, d), ref, f"step {step}")
        if step % 2:
            p += 1
    m.assert_ring_equal(0, 0)


@pytest.mark.parametrize("fused", [False, True])
def test_masked_slots_with_nonfinite_scales(gpu, fused):
    """Slots outside the window (and, fused, the current slot before the
    write) hold blocks with infinite and NaN scales: the output depends on
    the window only, so it stays finite and matches the oracle."""
    n_kv, d, n_ctx = 4, 128, 64
    m = Mirror(gpu, 1, 1, n_kv, d, n_ctx)
    pos = 20  # window 21 (fused: 20 ring keys + the new one); slots 21.. are outside
    m.fill_range(0, 0, 0, pos, seed=77)
    nblk = d // 32
    bad = np.zeros((n_ctx - pos, n_kv, nblk), dtype=oracle.BLOCK_DTYPE)
    bad["d"] = np.where(np.arange(n_ctx - pos)[:, None, None] % 2 == 0, 0x7C00, 0x7E00)  # inf / NaN
    bad["qs"] = 0x3C
    for which in (0, 1):
        m.ring.import_q4_0(0, 0, which, pos, bad.view(np.uint8))
    gpu.cuda.synchronize()
    n_heads = 8
    q = oracle.normal(78, n_heads * d)
    out = gpu.full((n_heads * d,), float("nan"), dtype=gpu.float32, device="cuda")
    posd = _i32(gpu, [pos])
    if fused:
        k = oracle.normal(79, n_kv * d)
        v = oracle.normal(80, n_kv * d)
        m.ring.append_decode(0, posd, m.dev(q), m.dev(k), m.dev(v), out, n_heads, stream=m.stream)
        m.oracle_append(0, 0, pos, k, v)
    else:
        m.oracle_append(0, 0, pos, oracle.normal(81, n_kv * d), oracle.normal(82, n_kv * d))
        kk = oracle.normal(81, n_kv * d)
        vv = oracle.normal(82, n_kv * d)
        m.ring.append(0, posd, m.dev(kk), m.dev(vv), stream=m.stream)
        m.ring.decode(0, posd, m.dev(q), out, n_heads, stream=m.stream)
    gpu.cuda.synchronize()
    got = out.cpu().numpy().reshape(n_heads, d)
    check_close(got, m.oracle_decode(0, 0, pos, q, n_heads), f"non-finite outside the window, fused={fused}")
