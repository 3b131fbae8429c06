"""The ggml-style CPU baseline (oracle/cpu_ggml_style.c: q to Q8_0, Q4_0 x
Q8_0 dot products, online softmax with expf, V dequantized to fp32) against an
independent numpy evaluation of the same steps: Q8_0 codes and fp16 scales of
q, exact integer block dots, float64 softmax over the ring window.  The SIMD
code keeps fp32 accumulators, so the bar is 2e-5 relative to the output's
scale.  Against the float64 oracle with fp32 q it differs by the Q8_0
rounding of q: about 1% of the output's norm, enough that some elements fall
outside the north-star bar 2e-3 + 1e-3 |ref| that the GPU decode meets (the
GPU path scores with fp32-accurate q; ggml's CPU backend would not)."""
import numpy as np
import pytest

import oracle


def _q8_0(x):
    x = x.reshape(-1, 32).astype(np.float32)
    amax = np.abs(x).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    idv = np.where(d != 0, (np.float32(1.0) / np.where(d != 0, d, 1)).astype(np.float32), 0)
    codes = np.round(x * idv[:, None]).astype(np.int64)  # roundf: halves away from zero
    halves = np.abs((x * idv[:, None]).astype(np.float32)) % 1 == 0.5
    codes = np.where(halves, (np.sign(x) * np.ceil(np.abs(x * idv[:, None]))).astype(np.int64), codes)
    return codes, d.astype(np.float16).astype(np.float64)


def _numpy_ggml_style(kc, vc, pos, q, n_heads):
    n_kv, n_ctx, nblk = kc.shape
    d = nblk * 32
    window = min(pos + 1, n_ctx)
    slots = [(pos + 1 - window + i) % n_ctx for i in range(window)]
    out = np.zeros((n_heads, d))
    for h in range(n_heads):
        kvh = h // (n_heads // n_kv)
        qc, qd = _q8_0(q[h])
        s = np.zeros(window)
        vrows = np.zeros((window, d))
        for i, sl in enumerate(slots):
            kb, vb = kc[kvh, sl], vc[kvh, sl]
            for b in range(nblk):
                codes = np.concatenate([kb["qs"][b] & 15, kb["qs"][b] >> 4]).astype(np.int64) - 8
                s[i] += float(np.float16(kb["d"][b].view(np.float16))) * qd[b] * int(codes @ qc[b])
                vcodes = np.concatenate([vb["qs"][b] & 15, vb["qs"][b] >> 4]).astype(np.float64) - 8
                vrows[i, b * 32:(b + 1) * 32] = vcodes * float(vb["d"][b].view(np.float16))
        s *= 1.0 / np.sqrt(np.float32(d))
        p = np.exp(s - s.max())
        out[h] = p @ vrows / p.sum()
    return out


@pytest.mark.parametrize("n_heads,n_kv,d,n_ctx,pos", [(4, 4, 128, 64, 100), (4, 2, 64, 40, 30),
                                                      (2, 2, 128, 512, 700)])
def test_ggml_style_matches_numpy(n_heads, n_kv, d, n_ctx, pos):
    kc, vc = oracle.new_ring(n_kv, n_ctx, d)
    lo = max(0, pos - n_ctx + 1)
    for p in range(lo, pos + 1):
        oracle.ring_append(kc, vc, p, oracle.normal(10 + p, n_kv * d), oracle.normal(20000 + p, n_kv * d))
    q = oracle.normal(7, n_heads * d).reshape(n_heads, d)
    secs, got = oracle.cpu_ggml_style_run(kc[None], vc[None], np.array([pos]), q[None], n_heads, 2, 1)
    ref = _numpy_ggml_style(kc, vc, pos, q, n_heads)
    scale = np.abs(ref).max()
    assert np.max(np.abs(got[0] - ref)) <= 2e-5 * scale
    f64 = oracle.ring_decode_f64(kc, vc, pos, q, n_heads)
    nrel = np.linalg.norm(got[0] - f64) / np.linalg.norm(f64)
    assert 1e-4 < nrel < 3e-2, nrel  # the Q8_0 rounding of q, and no more


def test_ggml_style_threads_agree():
    n_kv, d, n_ctx = 4, 128, 128
    n_sess = 3
    kc = np.zeros((n_sess, n_kv, n_ctx, d // 32), oracle.BLOCK_DTYPE)
    vc = np.zeros_like(kc)
    pos = np.array([200, 50, 127])
    for s in range(n_sess):
        for p in range(max(0, pos[s] - n_ctx + 1), pos[s] + 1):
            oracle.ring_append(kc[s], vc[s], p, oracle.normal(s * 1000 + p, n_kv * d),
                               oracle.normal(s * 1000 + 500 + p, n_kv * d))
    q = oracle.normal(9, n_sess * n_kv * d).reshape(n_sess, n_kv, d)
    _, one = oracle.cpu_ggml_style_run(kc, vc, pos, q, n_kv, 1, 1)
    _, many = oracle.cpu_ggml_style_run(kc, vc, pos, q, n_kv, 5, 2)
    assert np.array_equal(one, many)
