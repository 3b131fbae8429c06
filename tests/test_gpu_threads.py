"""Two host threads drive two rings at once, each on its own stream, through
the C ABI: fused append + decode steps on one, plain decode on the other,
while a third thread keeps making failing calls on a third ring.  Every
output matches the float64 oracle, the rings match it bit for bit, and the
failing calls' errors stay on their own ring (per-ring error state, the
registry of ring bases and the device guard are shared host state)."""
import threading

import numpy as np
import pytest

import oracle
from _ringsim import Mirror, check_close

pytestmark = pytest.mark.gpu


def _i32(torch, vals):
    return torch.tensor(list(vals), dtype=torch.int32, device="cuda")


def test_two_threads_two_rings(gpu):
    torch = gpu
    from bmo_jetson_amd import KVRing, RingError

    steps = 24
    ma = Mirror(torch, 1, 1, 4, 128, 64)   # fused append + decode, 4 heads x 128
    mb = Mirror(torch, 2, 1, 2, 64, 40)    # decode over a filled ring, 2 kv heads x 64, GQA 4:2
    mb.fill_range(1, 0, 0, 70, seed=5)
    nha, nhb = 4, 4
    qa = [oracle.normal(100 + i, nha * 128) for i in range(steps)]
    ka = [oracle.normal(200 + i, nha * 128) for i in range(steps)]
    va = [oracle.normal(300 + i, nha * 128) for i in range(steps)]
    qb = [oracle.normal(400 + i, nhb * 64) for i in range(steps)]
    dev = lambda m, xs: [m.dev(x) for x in xs]
    qa_d, ka_d, va_d, qb_d = dev(ma, qa), dev(ma, ka), dev(ma, va), dev(mb, qb)
    pa = [_i32(torch, [i]) for i in range(steps)]
    pb = _i32(torch, [69])
    outs = {"a": [], "b": []}
    errors = []

    def run_a():
        try:
            st = torch.cuda.Stream()
            out = torch.empty(nha * 128, device="cuda")
            for i in range(steps):
                ma.ring.append_decode(0, pa[i], qa_d[i], ka_d[i], va_d[i], out, nha, stream=st)
                st.synchronize()
                outs["a"].append(out.cpu().numpy().copy())
        except Exception as e:  # surfaced in the main thread
            errors.append(e)

    def run_b():
        try:
            st = torch.cuda.Stream()
            out = torch.empty(nhb * 64, device="cuda")
            for i in range(steps):
                mb.ring.decode(1, pb, qb_d[i], out, nhb, stream=st)
                st.synchronize()
                outs["b"].append(out.cpu().numpy().copy())
        except Exception as e:
            errors.append(e)

    bad = KVRing(1, 1, 2, 128, 16)
    bad_q = torch.zeros(2 * 128, device="cuda")
    bad_rc = []

    def run_bad():
        for _ in range(steps):
            try:
                bad.decode(3, pb, bad_q, bad_q, 2)     # layer out of range
            except RingError as e:
                bad_rc.append(e.rc)

    threads = [threading.Thread(target=f) for f in (run_a, run_b, run_bad)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a thread did not finish"
    assert not errors, errors
    assert bad_rc == [2] * steps
    assert bad.last_error() is not None
    assert ma.ring.last_error() is None and mb.ring.last_error() is None
    bad.close()

    for i in range(steps):
        ma.oracle_append(0, 0, i, ka[i], va[i])
        check_close(outs["a"][i].reshape(nha, 128), ma.oracle_decode(0, 0, i, qa[i], nha),
                    f"thread a, step {i}")
        check_close(outs["b"][i].reshape(nhb, 64), mb.oracle_decode(1, 0, 69, qb[i], nhb),
                    f"thread b, step {i}")
    ma.assert_ring_equal(0, 0)
    mb.assert_ring_equal(1, 0)
