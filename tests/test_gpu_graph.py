"""A whole decode step captured once into a HIP graph and replayed per token.

The step is what a model issues per token on the attention path: for every
layer the RoPE-fused append + decode (bmo_kv_ring_append_decode_rope), then
bmo_positions_advance.  The kernels read positions from device memory when
they run, so each replay rotates, appends and attends at the current
positions (the reference's static capture froze RoPE at the capture-time
position and was disabled, src/bmo_api.cpp:334-350).  Every replay is checked
against the oracle: ring bit-exact, outputs within 2e-3 + 1e-3 |ref|.  The
inputs are rewritten between replays by eager copies, and the replays are
separated by synchronizations, as a token loop would be."""
import numpy as np
import pytest

import oracle
from _ringsim import Mirror, check_close
from bmo_jetson_amd import positions_advance

pytestmark = pytest.mark.gpu


def _capture(gpu, launch):
    graph = gpu.cuda.CUDAGraph()
    s = gpu.cuda.Stream()
    s.wait_stream(gpu.cuda.current_stream())
    with gpu.cuda.stream(s):
        with gpu.cuda.graph(graph, stream=s):
            launch(gpu.cuda.current_stream())
    gpu.cuda.current_stream().wait_stream(s)
    gpu.cuda.synchronize()
    return graph


@pytest.mark.parametrize("theta", [10000.0, None])
def test_graph_replay_advances_positions(gpu, theta):
    L, S, H, n_kv, d, n_ctx = 3, 3, 8, 4, 128, 16
    m = Mirror(gpu, L, S, n_kv, d, n_ctx)
    start = [5, 0, 30]
    for s, p in enumerate(start):
        for layer in range(L):
            m.fill_range(layer, s, 0, p, seed=500 + 10 * s + layer)
    pos = gpu.tensor(start, dtype=gpu.int32, device="cuda")
    q = gpu.zeros((L, S, H, d), dtype=gpu.float32, device="cuda")
    k = gpu.zeros((L, S, n_kv, d), dtype=gpu.float32, device="cuda")
    v = gpu.zeros_like(k)
    out = gpu.zeros((L, S, H, d), dtype=gpu.float32, device="cuda")

    def step(st):
        for layer in range(L):
            m.ring.append_decode(layer, pos, q[layer], k[layer], v[layer], out[layer], H,
                                 stream=st, rope_theta=theta)
        positions_advance(pos, S, 1, stream=st)

    graph = _capture(gpu, step)
    cur = list(start)
    for t in range(20):
        qh = oracle.normal(1000 + t, L * S * H * d).reshape(L, S, H, d)
        kh = oracle.normal(2000 + t, L * S * n_kv * d).reshape(L, S, n_kv, d)
        vh = oracle.normal(3000 + t, L * S * n_kv * d).reshape(L, S, n_kv, d)
        q.copy_(gpu.from_numpy(qh))
        k.copy_(gpu.from_numpy(kh))
        v.copy_(gpu.from_numpy(vh))
        graph.replay()
        gpu.cuda.synchronize()
        got = out.cpu().numpy()
        for layer in range(L):
            for s in range(S):
                p = cur[s]
                kr = kh[layer, s] if theta is None else oracle.rope_interleaved(kh[layer, s], p, theta)
                qr = qh[layer, s] if theta is None else oracle.rope_interleaved(qh[layer, s], p, theta)
                m.oracle_append(layer, s, p, kr, vh[layer, s])
                check_close(got[layer, s], m.oracle_decode(layer, s, p, qr, H),
                            f"replay {t} layer {layer} session {s} pos {p}")
        cur = [p + 1 for p in cur]
        assert pos.cpu().tolist() == cur
    for layer in range(L):
        for s in range(S):
            m.assert_ring_equal(layer, s)
