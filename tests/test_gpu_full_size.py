"""BASELINE configs 3, 4 and 5 at their real sizes, checked against the oracle.

Each test runs the full-size launch exactly as bench.py times it, then checks
a fixed sample of sessions (every head of each) against the float64 oracle at
the north-star tolerance |gpu - ref| <= 2e-3 + 1e-3 |ref|, and the sampled
sessions' ring stripes byte for byte against the oracle's Q4_0 restatement:

  * config 3: 64 sessions x 32 heads x d128, W=512, positions ~U[512, 4096),
    K/V ~N(0,1) with each element scaled x8 with probability 1%; layer 31 of
    a 32-layer ring (4.83 GB), so stripe offsets reach 4.7 GB;
  * config 4: the same at 256 sessions with the fused append of the new fp32
    K/V rows; layer 31 of the 19.3 GB ring, offsets past 2^34;
  * config 5: chunked prefill of 16 sessions x 256 bf16 tokens x 32 heads
    into a W=512 ring, with the history full (pos0 = 1024) and empty (0).

K/V are generated on the GPU with a seeded torch generator; the sampled
sessions' rows are copied back and quantized by the oracle."""
import numpy as np
import pytest

import oracle
from _ringsim import check_close
from bmo_jetson_amd import KVRing

pytestmark = pytest.mark.gpu

H, D, W = 32, 128, 512
NBLK = D // 32


def _i32(torch, vals):
    return torch.tensor([int(v) for v in vals], dtype=torch.int32, device="cuda")


def _kv_rows(torch, gen, n, outliers):
    """n rows of [H][D] K and V on the GPU, ~N(0,1), optionally x8 w.p. 1%."""
    k = torch.randn((n, H, D), device="cuda", generator=gen)
    v = torch.randn((n, H, D), device="cuda", generator=gen)
    if outliers:
        k.mul_(torch.where(torch.rand((n, H, D), device="cuda", generator=gen) < 0.01, 8.0, 1.0))
        v.mul_(torch.where(torch.rand((n, H, D), device="cuda", generator=gen) < 0.01, 8.0, 1.0))
    return k, v


def _oracle_stripes(k_host, v_host, lo):
    """Oracle ring stripes [H][W][NBLK] holding rows of positions lo.. (at
    most W of them, the last W)."""
    kc, vc = oracle.new_ring(H, W, D)
    n = k_host.shape[0]
    slots = (lo + np.arange(n)) % W
    kq = oracle.quantize_q4_0(k_host.reshape(-1)).reshape(n, H, NBLK)
    vq = oracle.quantize_q4_0(v_host.reshape(-1)).reshape(n, H, NBLK)
    kc[:, slots, :] = kq.transpose(1, 0, 2)
    vc[:, slots, :] = vq.transpose(1, 0, 2)
    return kc, vc


def _assert_stripes_equal(ring, layer, s, kc, vc, what):
    for which, c in ((0, kc), (1, vc)):
        got = ring.export_q4_0(layer, s, which, 0, W)
        ref = np.ascontiguousarray(c.transpose(1, 0, 2)).view(np.uint8).reshape(got.shape)
        if not np.array_equal(got, ref):
            diff = np.argwhere(got != ref)
            raise AssertionError(f"{what}: ring {'KV'[which]} of session {s}: {len(diff)} bytes "
                                 f"differ, first at (slot, head, blk, byte)={tuple(diff[0])}")


def _decode_config(gpu, S, fused, seed, sample):
    torch = gpu
    L, layer = 32, 31
    rng = np.random.default_rng(seed)
    pos = rng.integers(512, 4096, size=S)
    ring = KVRing(L, S, H, D, W)
    try:
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed)
        stream = torch.cuda.current_stream()
        host = {}
        for s in range(S):
            # the window ending at pos (decode) or just before it (fused append)
            hi = int(pos[s]) + (0 if fused else 1)
            lo = hi - W if not fused else hi - (W - 1)
            k, v = _kv_rows(torch, gen, hi - lo, outliers=True)
            ring.write(layer, s, lo, k, v, stream=stream)
            if s in sample:
                host[s] = (lo, k.cpu().numpy(), v.cpu().numpy())
        q = torch.randn((S, H, D), device="cuda", generator=gen)
        out = torch.full((S, H, D), float("nan"), device="cuda")
        posd = _i32(torch, pos)
        if fused:
            kn = torch.randn((S, H, D), device="cuda", generator=gen)
            vn = torch.randn((S, H, D), device="cuda", generator=gen)
            ring.append_decode(layer, posd, q, kn, vn, out, H, stream=stream)
        else:
            ring.decode(layer, posd, q, out, H, stream=stream)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        qh = q.cpu().numpy()
        assert np.all(np.isfinite(got)), "non-finite output"
        for s in sample:
            lo, kh, vh = host[s]
            if fused:
                kh = np.concatenate([kh, kn[s].cpu().numpy()[None]])
                vh = np.concatenate([vh, vn[s].cpu().numpy()[None]])
            kc, vc = _oracle_stripes(kh, vh, lo)
            what = f"{'cfg4' if fused else 'cfg3'} session {s} pos {int(pos[s])}"
            _assert_stripes_equal(ring, layer, s, kc, vc, what)
            check_close(got[s], oracle.ring_decode_f64(kc, vc, int(pos[s]), qh[s], H), what)
    finally:
        ring.close()


def test_cfg3_full_size_decode(gpu):
    _decode_config(gpu, 64, False, 0xB0A00003, sample=[0, 1, 17, 31, 32, 45, 62, 63])


def test_cfg4_full_size_fused(gpu):
    _decode_config(gpu, 256, True, 0xB0A00004, sample=[0, 1, 100, 127, 128, 200, 254, 255])


@pytest.mark.parametrize("pos0", [1024, 0])
def test_cfg5_full_size_prefill(gpu, pos0):
    torch = gpu
    S, C = 16, 256
    sample = [0, 7, 15]
    ring = KVRing(1, S, H, D, W)
    try:
        gen = torch.Generator(device="cuda")
        gen.manual_seed(0xB0A00005 + pos0)
        stream = torch.cuda.current_stream()
        hist = {}
        if pos0:
            for s in range(S):
                k, v = _kv_rows(torch, gen, W, outliers=False)
                ring.write(0, s, pos0 - W, k, v, stream=stream)
                if s in sample:
                    hist[s] = (k.cpu().numpy(), v.cpu().numpy())
        q = torch.randn((S, C, H, D), device="cuda", generator=gen).to(torch.bfloat16)
        k = torch.randn((S, C, H, D), device="cuda", generator=gen).to(torch.bfloat16)
        v = torch.randn((S, C, H, D), device="cuda", generator=gen).to(torch.bfloat16)
        out = torch.full((S, C, H, D), float("nan"), device="cuda")
        ring.prefill(0, torch.full((S,), pos0, dtype=torch.int32, device="cuda"), q, k, v, out, H,
                     n_tok=C, stream=stream)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert np.all(np.isfinite(got)), "non-finite output"
        qf, kf, vf = (x.float().cpu().numpy() for x in (q, k, v))
        for s in sample:
            if pos0:
                kc, vc = _oracle_stripes(*hist[s], pos0 - W)
            else:
                kc, vc = oracle.new_ring(H, W, D)
            what = f"cfg5 pos0 {pos0} session {s}"
            ref = oracle.ring_prefill_f64(kc, vc, pos0, qf[s], kf[s], vf[s], H)
            check_close(got[s], ref, what)
            # after the chunk the ring holds the chunk's blocks at its slots
            kc2, vc2 = _oracle_stripes(kf[s], vf[s], pos0)
            if pos0:
                kc2h, vc2h = _oracle_stripes(*hist[s], pos0 - W)
                keep = np.ones(W, bool)
                keep[(pos0 + np.arange(C)) % W] = False
                kc2[:, keep], vc2[:, keep] = kc2h[:, keep], vc2h[:, keep]
            _assert_stripes_equal(ring, 0, s, kc2, vc2, what)
    finally:
        ring.close()
