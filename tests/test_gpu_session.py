"""GPU tests of the per-session handle (bmo_attn_session_*, the attention part
of the reference's bmo_handle, src/bmo_api.cpp:164-172), driven through the C
ABI with ctypes and checked against the oracle:

  * eager token steps (every layer's fused append + attention at one
    position) through several ring wraps; the position advances by one per
    step (h->pos = pos + 1, src/bmo_api.cpp:501);
  * a step captured into a HIP graph inside the library and replayed 20
    times with new inputs, with and without RoPE, including a jump to another
    position and eager steps between replays (the graph reads the device
    position; bmo_capture_graphs / bmo_has_cuda_graphs, :334-359);
  * reset (position 0, the session's K/V zeroed, bmo_reset :258-272);
  * argument errors and their messages;
  * two handles on two sessions of one ring driven from two host threads.

Every output is compared with the float64 oracle at |gpu - ref| <= 2e-3 +
1e-3 |ref| and the ring stripes byte for byte."""
import threading

import numpy as np
import pytest

import oracle
from _ringsim import Mirror, check_close
from bmo_jetson_amd import RingError, Session, lib

pytestmark = pytest.mark.gpu

L, S, H_KV, D, N_CTX = 3, 3, 2, 128, 16
H = 4


def _inputs(seed):
    q = oracle.normal(seed, L * H * D).reshape(L, H, D)
    k = oracle.normal(seed + 1, L * H_KV * D).reshape(L, H_KV, D)
    v = oracle.normal(seed + 2, L * H_KV * D).reshape(L, H_KV, D)
    return q, k, v


def _oracle_step(m, s, pos, q, k, v, theta):
    refs = []
    for layer in range(L):
        kk = oracle.rope_interleaved(k[layer], pos, theta) if theta else k[layer]
        m.oracle_append(layer, s, pos, kk, v[layer])
        qq = oracle.rope_interleaved(q[layer], pos, theta) if theta else q[layer]
        refs.append(m.oracle_decode(layer, s, pos, qq, H))
    return np.stack(refs)


def _bufs(gpu):
    q = gpu.zeros((L, H, D), dtype=gpu.float32, device="cuda")
    k = gpu.zeros((L, H_KV, D), dtype=gpu.float32, device="cuda")
    v = gpu.zeros((L, H_KV, D), dtype=gpu.float32, device="cuda")
    out = gpu.full((L, H, D), float("nan"), dtype=gpu.float32, device="cuda")
    return q, k, v, out


def _load(gpu, bufs, q, k, v):
    for dst, src in zip(bufs[:3], (q, k, v)):
        dst.copy_(gpu.from_numpy(src))
    bufs[3].fill_(float("nan"))
    gpu.cuda.synchronize()  # the handle runs on its own stream


def _assert_all_rings(m):
    for layer in range(L):
        for s in range(S):
            m.assert_ring_equal(layer, s)


@pytest.mark.parametrize("theta", [0.0, 10000.0])
def test_eager_steps_through_wraps(gpu, theta):
    m = Mirror(gpu, L, S, H_KV, D, N_CTX)
    sess = Session(m.ring, 1, H, rope_theta=theta)
    assert sess.pos == 0 and not sess.has_graph
    bufs = _bufs(gpu)
    for pos in range(2 * N_CTX + 5):
        q, k, v = _inputs(100 + pos)
        _load(gpu, bufs, q, k, v)
        sess.forward(pos, *bufs)
        assert sess.pos == pos + 1
        ref = _oracle_step(m, 1, pos, q, k, v, theta)
        check_close(bufs[3].cpu().numpy(), ref, f"eager step pos {pos} theta {theta}")
    _assert_all_rings(m)  # sessions 0 and 2 untouched
    sess.close()


@pytest.mark.parametrize("theta", [0.0, 10000.0])
def test_captured_step_replays(gpu, theta):
    m = Mirror(gpu, L, S, H_KV, D, N_CTX)
    sess = Session(m.ring, 2, H, rope_theta=theta)
    bufs = _bufs(gpu)
    # some history first, eagerly
    for pos in range(5):
        q, k, v = _inputs(300 + pos)
        _load(gpu, bufs, q, k, v)
        sess.forward(pos, *bufs)
        _oracle_step(m, 2, pos, q, k, v, theta)
    sess.capture(*bufs)
    assert sess.has_graph and sess.pos == 5  # capturing runs nothing
    _assert_all_rings(m)
    positions = list(range(5, 15)) + [1000, 1001, 1002] + list(range(1003, 1010))
    assert len(positions) == 20
    for i, pos in enumerate(positions):
        q, k, v = _inputs(400 + i)
        _load(gpu, bufs, q, k, v)
        if i == 12:
            # an eager step between replays, at the next position
            sess.forward(pos, *bufs)
        else:
            sess.replay(pos)
        assert sess.pos == pos + 1
        ref = _oracle_step(m, 2, pos, q, k, v, theta)
        check_close(bufs[3].cpu().numpy(), ref, f"replay {i} pos {pos} theta {theta}")
    _assert_all_rings(m)
    sess.close()


def test_reset(gpu):
    m = Mirror(gpu, L, S, H_KV, D, N_CTX)
    for s in range(S):
        for layer in range(L):
            m.fill_range(layer, s, 0, 20, seed=50 + s + 10 * layer)
    sess = Session(m.ring, 0, H)
    bufs = _bufs(gpu)
    q, k, v = _inputs(7)
    _load(gpu, bufs, q, k, v)
    sess.forward(20, *bufs)
    _oracle_step(m, 0, 20, q, k, v, 0.0)
    sess.reset()
    assert sess.pos == 0
    for layer in range(L):
        m.orc[(layer, 0)] = oracle.new_ring(H_KV, N_CTX, D)
    _assert_all_rings(m)  # session 0 zeroed, the others kept
    q, k, v = _inputs(8)
    _load(gpu, bufs, q, k, v)
    sess.forward(0, *bufs)
    check_close(bufs[3].cpu().numpy(), _oracle_step(m, 0, 0, q, k, v, 0.0), "after reset")
    assert sess.pos == 1
    sess.close()


def test_argument_errors(gpu):
    m = Mirror(gpu, L, S, H_KV, D, N_CTX)
    with pytest.raises(RuntimeError, match="session out of range"):
        Session(m.ring, S, H)
    with pytest.raises(RuntimeError, match="multiple"):
        Session(m.ring, 0, 3)
    with pytest.raises(RuntimeError, match="rope_theta"):
        Session(m.ring, 0, H, rope_theta=-1.0)
    sess = Session(m.ring, 0, H)
    bufs = _bufs(gpu)
    with pytest.raises(RingError) as e:
        sess.replay(0)
    assert e.value.rc == 2 and "capture" in sess.last_error()
    for bad in (-1, 2**31 - 1):
        with pytest.raises(RingError) as e:
            sess.forward(bad, *bufs)
        assert e.value.rc == 2 and "pos" in sess.last_error()
    rc = lib().bmo_attn_session_forward(sess.handle, 0, None, bufs[1].data_ptr(),
                                        bufs[2].data_ptr(), bufs[3].data_ptr())
    assert rc == 1
    assert lib().bmo_attn_session_reset(None) == 1 and lib().bmo_attn_session_pos(None) == -1
    assert sess.pos == 0  # failed calls leave the position
    _assert_all_rings(m)  # and the ring
    q, k, v = _inputs(9)
    _load(gpu, bufs, q, k, v)
    sess.forward(0, *bufs)  # a good call clears the message
    assert sess.last_error() is None
    sess.close()
    lib().bmo_attn_session_free(None)


def test_two_sessions_two_threads(gpu):
    m = Mirror(gpu, L, S, H_KV, D, N_CTX)
    sessions = {0: Session(m.ring, 0, H, rope_theta=10000.0), 2: Session(m.ring, 2, H)}
    n_steps = 12
    inputs = {s: [_inputs(1000 * (s + 1) + p) for p in range(n_steps)] for s in sessions}
    outs = {s: [] for s in sessions}
    bufs = {s: _bufs(gpu) for s in sessions}
    for s in sessions:
        for dst in bufs[s][:3]:
            dst.zero_()
    gpu.cuda.synchronize()
    errors = []

    def drive(s):
        try:
            sess, b = sessions[s], bufs[s]
            for p in range(n_steps):
                q, k, v = inputs[s][p]
                # host -> device on the handle's own stream through torch
                st = gpu.cuda.ExternalStream(sess.stream)
                with gpu.cuda.stream(st):
                    for dst, src in zip(b[:3], (q, k, v)):
                        dst.copy_(gpu.from_numpy(src))
                    st.synchronize()
                sess.forward(3 * p + s, *b)
                outs[s].append(b[3].cpu().numpy().copy())
        except Exception as ex:  # reported on the main thread
            errors.append(ex)

    threads = [threading.Thread(target=drive, args=(s,)) for s in sessions]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    for s, theta in ((0, 10000.0), (2, 0.0)):
        for p in range(n_steps):
            q, k, v = inputs[s][p]
            ref = _oracle_step(m, s, 3 * p + s, q, k, v, theta)
            check_close(outs[s][p], ref, f"thread session {s} step {p}")
        assert sessions[s].pos == 3 * (n_steps - 1) + s + 1
    _assert_all_rings(m)
    for sess in sessions.values():
        sess.close()
