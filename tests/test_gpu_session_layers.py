"""GPU tests of the per-session handle at a model's layer granularity
(bmo_attn_session_begin_step / _layer / _end_step / _reset_async / _sync /
_capture_begin / _capture_end), driven through the C ABI with ctypes.

The reference's layer loop (src/bmo_compute.cpp:2188-2641, driven by
bmo_forward_temporal2, src/bmo_api.cpp:384-511) computes layer l+1's q/k/v
from layer l's attention output through the projections (QKV at :2232,
output at :2423).  Here a 4-layer loop at the temporal shape (32 heads x
head_dim 128, a 512-slot ring with history, RoPE) feeds each layer's output
into the next layer's Q4_0 x Q8_1 QKV projection (bmo_launch_gemv_q4_0_q8_1)
on the handle's stream: two steps run eagerly, then the whole step -- four
projections and four attention layers -- is captured once and replayed 20
times with new inputs.  The depformer's frame (bmo_forward_depth_cascade,
src/bmo_api.cpp:668-743: a reset at :682, then 8 codebook steps x 6 layers,
16 heads x head_dim 64 on an 8-slot ring) is captured as one graph and
replayed for three frames.

Every stage is checked against the oracle on the GPU's own inputs to it:
each projection against the float64 GEMV of the GPU's activation (the
activation's Q8_1 exactly as the reference forms it), each attention output
against the float64 oracle at |gpu - ref| <= 2e-3 + 1e-3 |ref| after the
oracle ring appended the GPU's k/v, and the ring byte for byte."""
import numpy as np
import pytest

import oracle
from _ringsim import Mirror, check_close
from bmo_jetson_amd import RingError, Session, gemv_q4_0_q8_1

pytestmark = pytest.mark.gpu

THETA = 10000.0


def _check_gemv(w, x, got, rows, cols, what):
    ref, tabs = oracle.gemv_q4_0_q8_1_f64(w, oracle.quantize_q8_1(x), rows, cols)
    err = np.abs(got.astype(np.float64) - ref)
    bound = 1e-5 * tabs + 1e-6
    assert np.all(err <= bound), f"{what}: {int(np.sum(err > bound))} rows out of tolerance"


class _Model:
    """L layers of (QKV projection, attention) on one session of a ring."""

    def __init__(self, gpu, L, H, D, W, session, n_sessions, hist_to):
        self.gpu, self.L, self.H, self.D = gpu, L, H, D
        self.E = H * D
        self.m = Mirror(gpu, L, n_sessions, H, D, W)
        for layer in range(L):
            self.m.fill_range(layer, session, 0, hist_to, seed=900 + layer)
        self.session = session
        # weights ~N(0, 1/E) (times 1/64, exact), so activations stay O(1)
        self.w = [oracle.quantize_q4_0(oracle.normal(4000 + l, 3 * self.E * self.E) / 64.0)
                  for l in range(L)]
        self.wd = [gpu.from_numpy(w.view(np.uint8).copy()).cuda() for w in self.w]
        self.x0 = gpu.zeros(self.E, dtype=gpu.float32, device="cuda")
        self.qkv = gpu.zeros((L, 3 * self.E), dtype=gpu.float32, device="cuda")
        self.out = gpu.zeros((L, self.E), dtype=gpu.float32, device="cuda")
        self.sess = Session(self.m.ring, session, H, rope_theta=THETA)

    def enqueue_layers(self):
        """The step's layers on the handle's stream: layer l's QKV from the
        previous layer's output (x0 for layer 0), then its attention."""
        E, st = self.E, self.sess.stream
        for l in range(self.L):
            x = self.x0 if l == 0 else self.out[l - 1]
            gemv_q4_0_q8_1(self.wd[l], x, self.qkv[l], 3 * E, E, stream=st)
            self.sess.layer(l, self.qkv[l, :E], self.qkv[l, E:2 * E], self.qkv[l, 2 * E:],
                            self.out[l])

    def load_input(self, seed):
        self.x0.copy_(self.gpu.from_numpy(oracle.normal(seed, self.E)))
        self.out.fill_(float("nan"))
        self.gpu.cuda.synchronize()  # the handle runs on its own stream

    def check_step(self, pos, x0, check_gemv, what):
        E, H, D = self.E, self.H, self.D
        qkv = self.qkv.cpu().numpy()
        out = self.out.cpu().numpy()
        for l in range(self.L):
            x = x0 if l == 0 else out[l - 1]
            if check_gemv:
                _check_gemv(self.w[l], x, qkv[l], 3 * E, E, f"{what} layer {l} QKV")
            q = qkv[l, :E].reshape(H, D)
            k = qkv[l, E:2 * E].reshape(H, D)
            v = qkv[l, 2 * E:].reshape(H, D)
            self.m.oracle_append(l, self.session, pos, oracle.rope_interleaved(k, pos, THETA), v)
            ref = self.m.oracle_decode(l, self.session, pos, oracle.rope_interleaved(q, pos, THETA), H)
            check_close(out[l].reshape(H, D), ref, f"{what} layer {l} attention")


def test_layer_loop_eager_then_captured_replays(gpu):
    L, H, D, W, P0 = 4, 32, 128, 512, 700
    md = _Model(gpu, L, H, D, W, session=1, n_sessions=2, hist_to=P0)
    sess = md.sess
    # two eager steps, one layer at a time with the projections between
    for i, pos in enumerate((P0, P0 + 1)):
        x0 = oracle.normal(7000 + i, md.E)
        md.load_input(7000 + i)
        sess.begin_step(pos)
        md.enqueue_layers()
        sess.end_step()
        assert sess.pos == pos + 1          # reported as soon as it is queued
        sess.sync()
        md.check_step(pos, x0, True, f"eager step at {pos}")
    # the whole step captured once: projections and attention, 4 layers
    sess.capture_begin()
    md.enqueue_layers()
    sess.end_step()
    sess.capture_end()
    assert sess.has_graph and sess.pos == P0 + 2   # nothing ran
    for r in range(20):
        pos = P0 + 2 + r
        seed = 7100 + r
        x0 = oracle.normal(seed, md.E)
        md.load_input(seed)
        sess.replay(pos)
        assert sess.pos == pos + 1
        md.check_step(pos, x0, r in (0, 1, 19), f"replay {r} at {pos}")
    for l in range(L):
        md.m.assert_ring_equal(l, 1)
        md.m.assert_ring_equal(l, 0)         # the other session is untouched


def test_depformer_frame_captured(gpu):
    """Reset + 8 codebook steps x 6 layers as one graph (bmo_forward_depth_cascade)."""
    L, H, D, W, STEPS = 6, 16, 64, 8, 8
    m = Mirror(gpu, L, 1, H, D, W)
    sess = Session(m.ring, 0, H)
    q = gpu.zeros((STEPS, L, H * D), dtype=gpu.float32, device="cuda")
    k = gpu.zeros_like(q)
    v = gpu.zeros_like(q)
    out = gpu.zeros_like(q)
    sess.capture_begin()
    sess.reset_async()
    for s in range(STEPS):
        for l in range(L):
            sess.layer(l, q[s, l], k[s, l], v[s, l], out[s, l])
        sess.end_step()
    sess.capture_end()
    assert sess.has_graph and sess.pos == 0
    for frame in range(3):
        qh = oracle.normal(8000 + 10 * frame, STEPS * L * H * D).reshape(STEPS, L, H, D)
        kh = oracle.normal(8001 + 10 * frame, STEPS * L * H * D).reshape(STEPS, L, H, D)
        vh = oracle.normal(8002 + 10 * frame, STEPS * L * H * D).reshape(STEPS, L, H, D)
        for dst, src in ((q, qh), (k, kh), (v, vh)):
            dst.copy_(gpu.from_numpy(src.reshape(STEPS, L, H * D)))
        out.fill_(float("nan"))
        gpu.cuda.synchronize()
        sess.replay(0)
        assert sess.pos == STEPS
        got = out.cpu().numpy().reshape(STEPS, L, H, D)
        m.orc = {(l, 0): oracle.new_ring(H, W, D) for l in range(L)}  # the frame's reset
        for s in range(STEPS):
            for l in range(L):
                m.oracle_append(l, 0, s, kh[s, l], vh[s, l])
                check_close(got[s, l], m.oracle_decode(l, 0, s, qh[s, l], H),
                            f"frame {frame} step {s} layer {l}")
        for l in range(L):
            m.assert_ring_equal(l, 0)


def test_capture_errors_keep_previous_graph(gpu):
    L, H, D, W = 2, 4, 128, 32
    m = Mirror(gpu, L, 1, H, D, W)
    sess = Session(m.ring, 0, H)
    q = gpu.zeros((L, H, D), dtype=gpu.float32, device="cuda")
    k, v, out = gpu.zeros_like(q), gpu.zeros_like(q), gpu.zeros_like(q)
    with pytest.raises(RingError) as e:
        sess.capture_end()                       # nothing open
    assert e.value.rc == 2 and "no capture" in e.value.msg
    sess.capture(q, k, v, out)                   # a one-step graph to keep
    sess.capture_begin()
    for call in (lambda: sess.begin_step(3), lambda: sess.sync(), lambda: sess.forward(0, q, k, v, out),
                 lambda: sess.replay(0), lambda: sess.reset(), lambda: sess.capture_begin()):
        with pytest.raises(RingError) as e:
            call()
        assert e.value.rc == 2 and "capture" in e.value.msg
    with pytest.raises(RingError):
        sess.layer(L, q[0], k[0], v[0], out[0])  # layer out of range inside the capture
    with pytest.raises(RingError) as e:
        sess.capture_end()
    assert "previous graph is kept" in e.value.msg
    assert sess.has_graph
    # the kept one-step graph still runs correctly
    for pos in range(3):
        qh = oracle.normal(9000 + pos, L * H * D).reshape(L, H, D)
        kh = oracle.normal(9100 + pos, L * H * D).reshape(L, H, D)
        vh = oracle.normal(9200 + pos, L * H * D).reshape(L, H, D)
        for dst, src in ((q, qh), (k, kh), (v, vh)):
            dst.copy_(gpu.from_numpy(src))
        gpu.cuda.synchronize()
        sess.replay(pos)
        got = out.cpu().numpy()
        for l in range(L):
            m.oracle_append(l, 0, pos, kh[l], vh[l])
            check_close(got[l], m.oracle_decode(l, 0, pos, qh[l], H), f"kept graph pos {pos} layer {l}")
    assert sess.pos == 3
    sess.close()
