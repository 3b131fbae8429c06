"""GPU parity of bmo_launch_gemv_q4_0_q8_1 (the reference's Q4_0 x Q8_1 GEMV,
src/bmo_cuda_kernels.cu:529-711) against the oracle: the activation's Q8_1
blocks (written to the scratch) bit-exact, and every output within
|gpu - ref| <= 1e-5 * sum_b |term_b| + 1e-6 of the float64 evaluation (fp32
accumulation of the same exact integer dot products)."""
import ctypes

import numpy as np
import pytest

import oracle
from bmo_jetson_amd import _lib

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _run(gpu, rows, cols, x, seed, scratch=True):
    w = oracle.quantize_q4_0(oracle.normal(seed, rows * cols))
    wd = gpu.from_numpy(w.view(np.uint8).copy()).cuda()
    xd = gpu.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()
    y = gpu.full((rows,), float("nan"), dtype=gpu.float32, device="cuda")
    q8 = gpu.zeros(cols // 32 * 36, dtype=gpu.uint8, device="cuda") if scratch else None
    rc = _lib.lib().bmo_launch_gemv_q4_0_q8_1(_ptr(wd), _ptr(xd), _ptr(y), rows, cols,
                                              _ptr(q8) if scratch else None, None)
    assert rc == 0
    gpu.cuda.synchronize()
    xq = oracle.quantize_q8_1(x)
    ref, tabs = oracle.gemv_q4_0_q8_1_f64(w, xq, rows, cols)
    got = y.cpu().numpy().astype(np.float64)
    assert np.all(np.isfinite(got))
    err = np.abs(got - ref)
    bound = 1e-5 * tabs + 1e-6
    assert np.all(err <= bound), f"{int(np.sum(err > bound))} rows out of tolerance, worst {err.max():.3e}"
    if scratch:
        assert np.array_equal(q8.cpu().numpy(), xq.view(np.uint8)), "Q8_1 blocks differ from the oracle"
    return got


@pytest.mark.parametrize("rows,cols", [
    (12288, 4096),   # temporal QKV projection
    (4096, 4096),    # output projection
    (11264, 4096),   # gating linear in (reference bench shape)
    (4096, 5632),    # gating linear out (reference bench shape)
    (37, 11264),     # three pair iterations per lane, rows not a multiple of 32
    (1, 64),
    (16383, 4096),   # four two-row chunks per wave of the streaming kernel, odd rows
    (6001, 2048),    # waves with fewer chunks than others, a one-row last chunk
    (3, 192),        # three pairs per row: lanes past them idle
    (2049, 4096),    # one workgroup more than a round of chunks
    (16385, 4096),   # beyond four chunks per wave: the pair-walking kernel
    (8191, 5632),    # two 7-piece chunks per wave, two pairs per lane, odd rows
    (4096, 6144),    # the widest rows the streaming kernel takes
    (64, 4352),      # 4096 < cols: lanes past the row's 68 pairs idle in the second pass
])
def test_gemv_shapes(gpu, rows, cols):
    _run(gpu, rows, cols, oracle.normal(7 + cols, cols), seed=rows)


def test_gemv_activation_edge_blocks(gpu):
    """Zero blocks, halves that round away from zero, a dominant outlier and
    the reference bench's constant 0.5 row."""
    cols = 1024
    x = oracle.normal(3, cols).copy()
    x[0:32] = 0.0
    x[32:64] = np.linspace(-127, 127, 32, dtype=np.float32)          # d = 1: exact codes
    x[64:96] = (np.arange(32, dtype=np.float32) - 15.5) * np.float32(2.0)  # x/d = k + 0.5 ties
    x[96] = 1e4
    _run(gpu, 300, cols, x, seed=11)
    _run(gpu, 64, 4096, np.full(4096, 0.5, np.float32), seed=12)


def test_gemv_without_scratch_and_errors(gpu):
    _run(gpu, 100, 2048, oracle.normal(5, 2048), seed=13, scratch=False)
    L = _lib.lib()
    buf = gpu.zeros(4096, dtype=gpu.float32, device="cuda")
    p = _ptr(buf)
    assert L.bmo_launch_gemv_q4_0_q8_1(None, p, p, 4, 64, None, None) == 1
    assert L.bmo_launch_gemv_q4_0_q8_1(p, p, p, 4, 96, None, None) == 2      # not a multiple of 64
    assert L.bmo_launch_gemv_q4_0_q8_1(p, p, p, 0, 64, None, None) == 2
    off = ctypes.c_void_p(buf.data_ptr() + 4)                                 # x not 16-byte aligned
    assert L.bmo_launch_gemv_q4_0_q8_1(p, off, p, 4, 64, None, None) == 2
    assert L.bmo_launch_gemv_q4_0_q8_1(p, p, p, 4, 65536, None, None) == 2
    gpu.cuda.synchronize()


def _launch(gpu, wbytes, w_off, x, rows, cols):
    """y from a weight matrix placed w_off bytes into its device buffer."""
    wd = gpu.zeros(wbytes.size + 64, dtype=gpu.uint8, device="cuda")
    wd[w_off:w_off + wbytes.size] = gpu.from_numpy(wbytes).cuda()
    xd = gpu.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()
    y = gpu.full((rows,), float("nan"), dtype=gpu.float32, device="cuda")
    rc = _lib.lib().bmo_launch_gemv_q4_0_q8_1(ctypes.c_void_p(wd.data_ptr() + w_off), _ptr(xd), _ptr(y),
                                              rows, cols, None, None)
    assert rc == 0
    gpu.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("rows,cols", [(12288, 4096), (4095, 5632), (2049, 1024)])
def test_gemv_kernels_agree_bitwise(gpu, monkeypatch, rows, cols):
    """The streaming kernel and the pair-walking kernel share the quantizer
    and the pair product, so their outputs are equal bit for bit: a matrix
    at a 16-byte aligned address takes the streaming kernel, the same matrix
    4 bytes further (or BMO_GEMV_STREAM=0) the pair-walking one."""
    w = oracle.quantize_q4_0(oracle.normal(rows + cols, rows * cols)).view(np.uint8).copy()
    x = oracle.normal(31 + cols, cols)
    a = _launch(gpu, w, 0, x, rows, cols)
    b = _launch(gpu, w, 4, x, rows, cols)
    monkeypatch.setenv("BMO_GEMV_STREAM", "0")
    c = _launch(gpu, w, 0, x, rows, cols)
    assert np.all(np.isfinite(a))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
    ref, tabs = oracle.gemv_q4_0_q8_1_f64(w.view(oracle.BLOCK_DTYPE), oracle.quantize_q8_1(x), rows, cols)
    assert np.all(np.abs(a - ref) <= 1e-5 * tabs + 1e-6)
