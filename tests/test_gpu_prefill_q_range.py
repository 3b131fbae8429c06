"""GPU parity of chunked prefill for queries with a wide dynamic range.

The reference scores keys with fp32 q (src/bmo_compute.cpp:2410-2412 hands
fp32 q to ggml_flash_attn_ext; src/bmo_cuda_kernels.cu:772-776).  Prefill
takes bf16 q into fp16 matrix instructions.  Two fp16
roundings would break the bar |gpu - ref| <= 2e-3 + 1e-3 |ref| against the
float64 oracle once q has large elements: q * scale * log2(e) rounded to 11
bits, and the dequantized key (c - 8) * d rounded to 11 bits (a CPU model of
both, D=128, 512 keys: 1-3% of query rows out of tolerance, up to 57x the
bound, for one x30..x1000 outlier channel per block).  The kernel therefore
scales each query row by a power of two (exact in fp16) and applies the
residual query factor to the fp32 scores, and feeds the key codes (c - 8)
exactly, each block's d multiplying its product in fp32.  These tests run the query kinds of the decode range tests
through prefill:

  * one outlier channel per 32-element block at x30, x100, x300, x1000 and
    x10000;
  * one outlier channel per query row at x300;
  * blocks mixing magnitudes 1e-3 and 1e3 element by element;
  * whole rows scaled by 2^20 (beyond fp16 after any fixed scaling), 2^-20
    and 2^-100;
  * rows whose blocks differ in scale by 2^30 from block to block;
  * keys scaled by 2^-11 .. 2^-20 (fp16 block scales down to subnormal) or
    2^8, with queries scaled to keep the scores' spread;

at config 5's head shape (32 heads x d128, a 512-slot ring with full history,
256-token chunks: the direct path), on the staged path with 4 query heads per
kv head, and in 12 seeded random shapes; a query row holding a NaN or an
infinity must come out NaN while every other row stays within tolerance.
The ring must match the oracle byte for byte after each chunk."""
import numpy as np
import pytest

import oracle
from _ringsim import Mirror, check_close

pytestmark = pytest.mark.gpu

KINDS = ["block_x30", "block_x100", "block_x300", "block_x1000", "block_x10000", "row_x300",
         "mixed_1e3", "row_2p20", "row_2m20", "row_2m100", "block_ramp_2p30"]


def _i32(torch, vals):
    return torch.tensor(list(vals), dtype=torch.int32, device="cuda")


def q_rows(kind, shape, seed):
    """bf16-representable query rows (fp32 array of `shape`, last axis d)
    with the named dynamic range, row by row."""
    d = shape[-1]
    rows = int(np.prod(shape[:-1]))
    rng = np.random.default_rng(seed)
    q = oracle.normal(seed, rows * d).reshape(rows, d).astype(np.float64)
    nblk = d // 32
    if kind.startswith("block_x"):
        f = float(kind[len("block_x"):])
        cols = np.arange(nblk) * 32 + rng.integers(0, 32, (rows, nblk))
        np.put_along_axis(q, cols, np.take_along_axis(q, cols, 1) * f, 1)
    elif kind == "row_x300":
        cols = rng.integers(0, d, (rows, 1))
        np.put_along_axis(q, cols, np.take_along_axis(q, cols, 1) * 300.0, 1)
    elif kind == "mixed_1e3":
        q *= np.where(rng.random((rows, d)) < 0.5, 1e-3, 1e3)
    elif kind == "row_2p20":
        q *= 2.0 ** 20
    elif kind == "row_2m20":
        q *= 2.0 ** -20
    elif kind == "row_2m100":
        q *= 2.0 ** -100
    elif kind == "block_ramp_2p30":
        for b in range(nblk):
            q[:, b * 32:(b + 1) * 32] *= 2.0 ** (30 * b / max(1, nblk - 1) - 15)
    else:
        raise ValueError(kind)
    return oracle.round_bf16(q.astype(np.float32)).reshape(shape)


def _bf16_normals(seed, shape):
    return oracle.round_bf16(oracle.normal(seed, int(np.prod(shape)))).reshape(shape)


def _prefill(gpu, m, layer, sids, pos0, q, k, v, n_heads, q_ref=None):
    """Runs one prefill call over entries (session sids[b], pos0[b]) and the
    oracle's over the same ring state, which also appends the chunk to the
    oracle ring (orc_ring_prefill_f64); returns the GPU output
    [n_batch][n_tok][n_heads][d] and the oracle's.  q_ref, if given, is the
    query the oracle sees instead of q."""
    n_batch, n_tok = q.shape[0], q.shape[1]
    out = gpu.full(q.shape, float("nan"), dtype=gpu.float32, device="cuda")
    m.ring.prefill(layer, _i32(gpu, pos0), m.dev(q, gpu.bfloat16), m.dev(k, gpu.bfloat16),
                   m.dev(v, gpu.bfloat16), out, n_heads, n_tok=n_tok,
                   session_ids=_i32(gpu, sids), stream=m.stream)
    gpu.cuda.synchronize()
    got = out.cpu().numpy()
    qr = q if q_ref is None else q_ref
    refs = []
    for b, (s, p0) in enumerate(zip(sids, pos0)):
        kc, vc = m.orc[(layer, s)]
        refs.append(oracle.ring_prefill_f64(kc, vc, p0, qr[b], k[b], v[b], n_heads))
    return got, np.stack(refs)


@pytest.mark.parametrize("kind", KINDS)
def test_prefill_cfg5_heads_q_range(gpu, kind):
    """Config 5's per-session shape: 32 heads x d128, W=512, history full,
    a 256-token chunk (direct path)."""
    n_heads, d, n_ctx, pos0, n_tok = 32, 128, 512, 1000, 256
    m = Mirror(gpu, 1, 1, n_heads, d, n_ctx)
    m.fill_range(0, 0, 0, pos0, seed=0xC5000 + KINDS.index(kind))
    q = q_rows(kind, (1, n_tok, n_heads, d), 0xC5100 + KINDS.index(kind))
    k = _bf16_normals(0xC5200, (1, n_tok, n_heads, d))
    v = _bf16_normals(0xC5300, (1, n_tok, n_heads, d))
    got, ref = _prefill(gpu, m, 0, [0], [pos0], q, k, v, n_heads)
    check_close(got, ref, f"prefill cfg5 heads q={kind}")
    m.assert_ring_equal(0, 0)


@pytest.mark.parametrize("kind", KINDS)
def test_prefill_staged_gqa_q_range(gpu, kind):
    """The staged path (stage, attention, commit): 16 query heads on 4 kv
    heads, W=512, history full, 256 tokens, two sessions."""
    n_heads, n_kv, d, n_ctx, n_tok = 16, 4, 128, 512, 256
    sids, pos0 = [1, 0], [1537, 700]   # entries in reverse session order
    m = Mirror(gpu, 1, 2, n_kv, d, n_ctx)
    for b, (s, p) in enumerate(zip(sids, pos0)):
        m.fill_range(0, s, 0, p, seed=0x6A000 + 10 * KINDS.index(kind) + b)
    q = q_rows(kind, (2, n_tok, n_heads, d), 0x6A100 + KINDS.index(kind))
    k = _bf16_normals(0x6A200, (2, n_tok, n_kv, d))
    v = _bf16_normals(0x6A300, (2, n_tok, n_kv, d))
    got, ref = _prefill(gpu, m, 0, sids, pos0, q, k, v, n_heads)
    check_close(got, ref, f"prefill staged GQA q={kind}")
    for s in sids:
        m.assert_ring_equal(0, s)


@pytest.mark.parametrize("seed", list(range(12)))
def test_prefill_random_shape_q_range(gpu, seed):
    """Random shapes (head_dim, ring size on and off the 32-slot grid,
    history, chunk length, query heads per kv head) with every entry's q
    drawn from one of the wide-range kinds."""
    r = np.random.default_rng(0xB0A0F100 + seed)
    d = int(r.choice([64, 128]))
    n_ctx = int(r.choice([24, 32, 40, 64, 96, 128, 256, 512]))
    n_kv = int(r.choice([1, 2]))
    n_heads = n_kv * int(r.choice([1, 1, 2, 4]))
    n_tok = int(r.integers(1, min(n_ctx, 256) + 1))
    n_sess = int(r.integers(1, 3))
    sids = [int(s) for s in r.permutation(n_sess)]
    pos0 = [int(r.choice([0, int(r.integers(1, n_ctx)), int(r.integers(n_ctx, 6 * n_ctx))]))
            for _ in sids]
    m = Mirror(gpu, 1, n_sess, n_kv, d, n_ctx)
    for b, (s, p) in enumerate(zip(sids, pos0)):
        m.fill_range(0, s, 0, p, seed=7000 + 31 * seed + b)
    kinds = [KINDS[int(r.integers(len(KINDS)))] for _ in sids]
    q = np.stack([q_rows(kinds[b], (n_tok, n_heads, d), 7100 + 17 * seed + b)
                  for b in range(n_sess)])
    k = _bf16_normals(7200 + seed, (n_sess, n_tok, n_kv, d))
    v = _bf16_normals(7300 + seed, (n_sess, n_tok, n_kv, d))
    got, ref = _prefill(gpu, m, 0, sids, pos0, q, k, v, n_heads)
    for b, (s, p) in enumerate(zip(sids, pos0)):
        what = (f"seed {seed} entry {b} q={kinds[b]} session {s} pos0 {p} n_tok {n_tok} d {d} "
                f"n_ctx {n_ctx} heads {n_heads}/{n_kv}")
        check_close(got[b], ref[b], what)
        m.assert_ring_equal(0, s)


# (key exponent, query exponent): keys N(0,1) * 2^ke, queries N(0,1) * 2^qe,
# so the scores keep a spread of about 6 log2 units while the blocks' fp16
# scales d run from normal through subnormal (ke -16, -20) to large (ke 8).
KEY_RANGES = [(-11, 13), (-16, 18), (-20, 22), (8, -6)]


@pytest.mark.parametrize("ke,qe", KEY_RANGES)
@pytest.mark.parametrize("n_kv", [32, 8])
def test_prefill_key_scale_range(gpu, ke, qe, n_kv):
    """Keys whose Q4_0 scales are subnormal in fp16, or large, against
    queries scaled so that the scores still matter: each block's d must
    reach the scores exactly (a flushed subnormal scale zeroes its keys, and
    a d carried at reduced precision moves the scores by up to 2^-8 of their
    size, far past the tolerance here).
    n_kv 32: config 5's head shape on the direct path; n_kv 8: 4 query heads
    per kv head on the staged path.  History full, 256-token chunk."""
    n_heads, d, n_ctx, pos0, n_tok = 32, 128, 512, 1000, 256
    m = Mirror(gpu, 1, 1, n_kv, d, n_ctx)
    lo = pos0 - n_ctx
    hk = oracle.normal(0x5CA10 + ke, n_ctx * n_kv * d).reshape(n_ctx, n_kv, d) * np.float32(2.0 ** ke)
    hv = oracle.normal(0x5CA20 + ke, n_ctx * n_kv * d).reshape(n_ctx, n_kv, d)
    m.write(0, 0, lo, hk.astype(np.float32), hv)
    q = oracle.round_bf16(_bf16_normals(0x5CA30, (1, n_tok, n_heads, d)) * np.float32(2.0 ** qe))
    k = oracle.round_bf16(_bf16_normals(0x5CA40, (1, n_tok, n_kv, d)) * np.float32(2.0 ** ke))
    v = _bf16_normals(0x5CA50, (1, n_tok, n_kv, d))
    got, ref = _prefill(gpu, m, 0, [0], [pos0], q, k, v, n_heads)
    check_close(got, ref, f"prefill key scale 2^{ke}, q 2^{qe}, n_kv {n_kv}")
    m.assert_ring_equal(0, 0)


@pytest.mark.parametrize("bad", [float("nan"), float("inf"), float("-inf")])
@pytest.mark.parametrize("n_kv", [4, 1])
def test_prefill_nonfinite_q_gives_nan_row(gpu, bad, n_kv):
    """A non-finite q element makes that query row (token, head) NaN, as fp32
    scoring would; every other row and the ring are unaffected.  n_kv 4: the
    direct path; n_kv 1 (4 query heads on one kv head): the staged path."""
    n_heads, d, n_ctx, pos0, n_tok = 4, 128, 128, 300, 48
    m = Mirror(gpu, 1, 1, n_kv, d, n_ctx)
    m.fill_range(0, 0, 0, pos0, seed=0xBAD0)
    q = _bf16_normals(0xBAD1, (1, n_tok, n_heads, d))
    k = _bf16_normals(0xBAD2, (1, n_tok, n_kv, d))
    v = _bf16_normals(0xBAD3, (1, n_tok, n_kv, d))
    q[0, 17, 2, 77] = bad
    q_ok = q.copy()
    q_ok[0, 17, 2] = 0.0
    got, ref = _prefill(gpu, m, 0, [0], [pos0], q, k, v, n_heads, q_ref=q_ok)
    assert np.all(np.isnan(got[0, 17, 2])), "row with a non-finite q must be NaN"
    mask = np.ones((n_tok, n_heads), bool)
    mask[17, 2] = False
    check_close(got[0][mask], ref[0][mask], "finite rows")
    m.assert_ring_equal(0, 0)
