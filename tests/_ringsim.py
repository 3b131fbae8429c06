"""Test helper: a GPU KVRing driven through the C ABI together with its CPU
oracle twin, plus the tolerance check used by every attention parity test.

Tolerance: |gpu - ref| <= 2e-3 + 1e-3 * |ref|
elementwise against the float64 oracle over the same Q4_0 blocks."""
from __future__ import annotations

import numpy as np

import oracle
from bmo_jetson_amd import KVRing

ATOL = 2e-3
RTOL = 1e-3


def check_close(got, ref, what="", atol=ATOL, rtol=RTOL):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    max_abs = float(err.max()) if err.size else 0.0
    nrel = float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))
    bad = int(np.count_nonzero(err > bound))
    assert bad == 0, f"{what}: {bad} elements out of tolerance, max_abs={max_abs:.3e}, norm_rel={nrel:.3e}"
    return max_abs, nrel


class Mirror:
    """GPU ring + oracle stripes ([layer][session] -> (kc, vc))."""

    def __init__(self, torch, n_layers, n_sessions, n_kv, d, n_ctx):
        self.torch = torch
        self.ring = KVRing(n_layers, n_sessions, n_kv, d, n_ctx)
        self.n_layers, self.n_sessions, self.n_kv, self.d, self.n_ctx = (
            n_layers, n_sessions, n_kv, d, n_ctx)
        self.orc = {(l, s): oracle.new_ring(n_kv, n_ctx, d)
                    for l in range(n_layers) for s in range(n_sessions)}

    def dev(self, a, dtype=None):
        t = self.torch.from_numpy(np.ascontiguousarray(a))
        if dtype is not None:
            t = t.to(dtype)
        return t.cuda()

    @property
    def stream(self):
        return self.torch.cuda.current_stream()

    def write(self, layer, session, pos0, k, v):
        """k, v: numpy [n_tok][n_kv][d] fp32."""
        self.ring.write(layer, session, pos0, self.dev(k), self.dev(v), stream=self.stream)
        kc, vc = self.orc[(layer, session)]
        for i in range(k.shape[0]):
            oracle.ring_append(kc, vc, pos0 + i, k[i], v[i])

    def fill_range(self, layer, session, lo, hi, seed):
        """Writes positions max(lo, hi - n_ctx) .. hi-1 from seeded normals."""
        lo = max(lo, hi - self.n_ctx, 0)
        n = hi - lo
        if n <= 0:
            return
        k = oracle.normal(seed, n * self.n_kv * self.d).reshape(n, self.n_kv, self.d)
        v = oracle.normal(seed + 1, n * self.n_kv * self.d).reshape(n, self.n_kv, self.d)
        self.write(layer, session, lo, k, v)

    def oracle_append(self, layer, session, pos, k, v):
        kc, vc = self.orc[(layer, session)]
        oracle.ring_append(kc, vc, pos, k, v)

    def oracle_decode(self, layer, session, pos, q, n_heads):
        kc, vc = self.orc[(layer, session)]
        return oracle.ring_decode_f64(kc, vc, pos, q, n_heads)

    def assert_ring_equal(self, layer, session):
        """Bit-exact comparison of the GPU ring's K and V blocks with the oracle."""
        kc, vc = self.orc[(layer, session)]
        for which, c in ((0, kc), (1, vc)):
            got = self.ring.export_q4_0(layer, session, which, 0, self.n_ctx)
            ref = np.ascontiguousarray(c.transpose(1, 0, 2)).view(np.uint8).reshape(got.shape)
            if not np.array_equal(got, ref):
                diff = np.argwhere(got != ref)
                raise AssertionError(
                    f"ring {'KV'[which]} layer {layer} session {session}: "
                    f"{len(diff)} bytes differ, first at (slot, head, blk, byte)={tuple(diff[0])}")
