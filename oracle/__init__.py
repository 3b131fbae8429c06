"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.  The
product package (bmo_jetson_amd) never imports it.

Ring stripe arrays used here follow the reference's ggml order
[n_heads][n_ctx][head_dim/32] of 18-byte Q4_0 blocks (BLOCK_DTYPE).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

BLOCK_DTYPE = np.dtype([("d", "<u2"), ("qs", "u1", (16,))])
assert BLOCK_DTYPE.itemsize == 18

_lib = None


def build(force: bool = True) -> str:
    """Compile liboracle.so with oracle/Makefile."""
    args = ["make", "-C", HERE]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.isfile(LIB_PATH):
            build(force=False)
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        i32, i64, u64, f64 = ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_double
        sig = {
            "orc_fp32_to_fp16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_fp16_to_fp32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_selftest_fp16_exhaustive": (i64, []),
            "orc_quantize_row_q4_0": (None, [P, P, i64]),
            "orc_dequantize_row_q4_0": (None, [P, P, i64]),
            "orc_ring_window": (None, [i64, i32, P, P, P]),
            "orc_ring_append": (None, [P, P, i32, i32, i32, i64, P, P]),
            "orc_ring_decode_f64": (None, [P, P, i32, i32, i32, i32, i64, P, f64, P]),
            "orc_ring_prefill_f64": (None, [P, P, i32, i32, i32, i32, i64, i32, P, P, P, f64, P]),
            "orc_ring_copy_k_f32": (None, [P, i32, i32, i32, i32, i32, P]),
            "orc_quantize_row_q8_1_bmo": (None, [P, P, i64]),
            "orc_vec_dot_q4_0_q8_1_f64": (f64, [P, P, i64]),
            "orc_gemv_q4_0_q8_1_f64": (None, [P, P, i32, i32, P]),
            "orc_gemv_term_abs_f64": (None, [P, P, i32, i32, P]),
            "orc_rope_freq": (f64, [f64, i32]),
            "orc_rope_cos_sin": (None, [i32, i64, f64, P, P]),
            "orc_rope_interleaved": (None, [P, P, i32, i32, i64, f64]),
            "orc_mix64": (u64, [u64]),
            "orc_fill_normal": (None, [u64, u64, P, i64]),
            "orc_fill_kv": (None, [u64, u64, P, i64]),
            "orc_synth_ln": (f64, [f64]),
            "orc_synth_cos2pi": (f64, [f64]),
            "orc_fill_u64": (None, [u64, u64, P, i64]),
            "orc_round_bf16": (ctypes.c_float, [ctypes.c_float]),
            "orc_cpu_decode_f32": (None, [P, P, i32, i32, i32, i32, i64, P, P, P]),
            "orc_cpu_baseline_run": (f64, [P, P, i32, i32, i32, i32, i32, P, P, P, i32, i32]),
            "orc_cpu_ggml_style_run": (f64, [P, P, i32, i32, i32, i32, i32, P, P, P, i32, i32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---- fp16 -------------------------------------------------------------------

def fp32_to_fp16_bits(x: float) -> int:
    return int(lib().orc_fp32_to_fp16(ctypes.c_float(x)))


def fp16_bits_to_fp32(h: int) -> float:
    return float(lib().orc_fp16_to_fp32(ctypes.c_uint16(h)))


def selftest_fp16_exhaustive() -> int:
    return int(lib().orc_selftest_fp16_exhaustive())


# ---- Q4_0 -------------------------------------------------------------------

def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    """fp32 array (size multiple of 32) -> array of BLOCK_DTYPE."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert x.size % 32 == 0
    out = np.zeros(x.size // 32, dtype=BLOCK_DTYPE)
    lib().orc_quantize_row_q4_0(_p(x), _p(out), x.size)
    return out


def dequantize_q4_0(blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks).reshape(-1)
    assert blocks.dtype == BLOCK_DTYPE
    out = np.zeros(blocks.size * 32, dtype=np.float32)
    lib().orc_dequantize_row_q4_0(_p(blocks), _p(out), out.size)
    return out


# ---- ring -------------------------------------------------------------------

def ring_window(pos: int, n_ctx: int):
    w = ctypes.c_int()
    s = ctypes.c_int64()
    c = ctypes.c_int()
    lib().orc_ring_window(pos, n_ctx, ctypes.byref(w), ctypes.byref(s), ctypes.byref(c))
    return w.value, s.value, c.value


def new_ring(n_kv_heads: int, n_ctx: int, head_dim: int):
    """Zeroed K and V stripe sets [n_kv_heads][n_ctx][head_dim/32] blocks."""
    shape = (n_kv_heads, n_ctx, head_dim // 32)
    return np.zeros(shape, dtype=BLOCK_DTYPE), np.zeros(shape, dtype=BLOCK_DTYPE)


def ring_append(kc, vc, pos: int, k: np.ndarray, v: np.ndarray) -> None:
    n_kv, n_ctx, nblk = kc.shape
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    assert k.size == n_kv * nblk * 32 and v.size == k.size
    lib().orc_ring_append(_p(kc), _p(vc), n_kv, nblk * 32, n_ctx, pos, _p(k), _p(v))


def ring_decode_f64(kc, vc, pos: int, q: np.ndarray, n_heads: int, scale=None) -> np.ndarray:
    n_kv, n_ctx, nblk = kc.shape
    d = nblk * 32
    q = np.ascontiguousarray(q, dtype=np.float32)
    assert q.size == n_heads * d
    if scale is None:
        scale = 1.0 / np.sqrt(np.float32(d), dtype=np.float32)
    out = np.zeros((n_heads, d), dtype=np.float64)
    lib().orc_ring_decode_f64(_p(kc), _p(vc), n_heads, n_kv, d, n_ctx, pos, _p(q),
                              float(scale), _p(out))
    return out


def ring_prefill_f64(kc, vc, pos0: int, q, k, v, n_heads: int, scale=None) -> np.ndarray:
    n_kv, n_ctx, nblk = kc.shape
    d = nblk * 32
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    n_tok = q.size // (n_heads * d)
    assert q.size == n_tok * n_heads * d and k.size == n_tok * n_kv * d and v.size == k.size
    assert n_tok <= n_ctx
    if scale is None:
        scale = 1.0 / np.sqrt(np.float32(d), dtype=np.float32)
    out = np.zeros((n_tok, n_heads, d), dtype=np.float64)
    lib().orc_ring_prefill_f64(_p(kc), _p(vc), n_heads, n_kv, d, n_ctx, pos0, n_tok,
                               _p(q), _p(k), _p(v), float(scale), _p(out))
    return out


def ring_copy_k_f32(kc, t_start: int, n_pos: int) -> np.ndarray:
    n_kv, n_ctx, nblk = kc.shape
    d = nblk * 32
    out = np.zeros((n_pos, n_kv, d), dtype=np.float32)
    lib().orc_ring_copy_k_f32(_p(kc), n_kv, d, n_ctx, t_start, n_pos, _p(out))
    return out


# ---- Q4_0 x Q8_1 GEMV -------------------------------------------------------

Q8_1 = np.dtype([("d", "<u2"), ("s", "<u2"), ("qs", "i1", (32,))])


def quantize_q8_1(x: np.ndarray) -> np.ndarray:
    """fp32 row (multiple of 32) -> the reference's Q8_1 blocks (36 bytes each)."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros(x.size // 32, dtype=Q8_1)
    lib().orc_quantize_row_q8_1_bmo(_p(x), out.ctypes.data, x.size)
    return out


def gemv_q4_0_q8_1_f64(w_blocks: np.ndarray, xq: np.ndarray, rows: int, cols: int):
    """w_blocks: [rows * cols/32] Q4_0 blocks (ggml AoS); xq: Q8_1 blocks.
    Returns (y, term_abs), both float64 [rows]."""
    w = np.ascontiguousarray(w_blocks)
    y = np.zeros(rows, dtype=np.float64)
    t = np.zeros(rows, dtype=np.float64)
    lib().orc_gemv_q4_0_q8_1_f64(w.ctypes.data, xq.ctypes.data, rows, cols, _p(y))
    lib().orc_gemv_term_abs_f64(w.ctypes.data, xq.ctypes.data, rows, cols, _p(t))
    return y, t


# ---- RoPE -------------------------------------------------------------------

def rope_freq(r: float, i: int) -> float:
    return lib().orc_rope_freq(r, i)


def rope_cos_sin(head_dim: int, pos: int, theta: float = 10000.0):
    cs = np.empty(head_dim // 2, dtype=np.float32)
    sn = np.empty(head_dim // 2, dtype=np.float32)
    lib().orc_rope_cos_sin(head_dim, pos, theta, _p(cs), _p(sn))
    return cs, sn


def rope_interleaved(x: np.ndarray, pos: int, theta: float = 10000.0) -> np.ndarray:
    """x: [..., head_dim] fp32 -> the rotated copy (interleaved pairs)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    d = x.shape[-1]
    y = np.empty_like(x)
    lib().orc_rope_interleaved(_p(x), _p(y), x.size // d, d, pos, theta)
    return y


# ---- synthetic inputs -------------------------------------------------------

def normal(seed: int, n: int, offset: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal(seed & (2**64 - 1), offset, _p(out), n)
    return out


def kv_normal(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """normal(), each element x8 with probability 1% (configurations 3, 4)."""
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_kv(seed & (2**64 - 1), offset, _p(out), n)
    return out


def words(seed: int, n: int, offset: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint64)
    lib().orc_fill_u64(seed & (2**64 - 1), offset, _p(out), n)
    return out


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to bf16 (returned as fp32), nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32).reshape(np.shape(x))


# ---- CPU baseline -----------------------------------------------------------

def cpu_decode_f32(kc, vc, pos: int, q: np.ndarray, n_heads: int) -> np.ndarray:
    n_kv, n_ctx, nblk = kc.shape
    d = nblk * 32
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros((n_heads, d), dtype=np.float32)
    scratch = np.zeros(n_ctx, dtype=np.float32)
    lib().orc_cpu_decode_f32(_p(kc), _p(vc), n_heads, n_kv, d, n_ctx, pos, _p(q), _p(out),
                             _p(scratch))
    return out


def cpu_baseline_run(kc, vc, pos: np.ndarray, q: np.ndarray, n_heads: int,
                     n_threads: int, iters: int):
    """kc, vc: [n_sess][n_kv][n_ctx][nblk] blocks; pos: int64[n_sess];
    q: [n_sess][n_heads][d].  Returns (seconds, out)."""
    n_sess, n_kv, n_ctx, nblk = kc.shape
    d = nblk * 32
    pos = np.ascontiguousarray(pos, dtype=np.int64)
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros((n_sess, n_heads, d), dtype=np.float32)
    secs = lib().orc_cpu_baseline_run(_p(kc), _p(vc), n_sess, n_heads, n_kv, d, n_ctx,
                                      _p(pos), _p(q), _p(out), n_threads, iters)
    return float(secs), out


def cpu_ggml_style_run(kc, vc, pos: np.ndarray, q: np.ndarray, n_heads: int,
                       n_threads: int, iters: int):
    """The ggml-style SIMD baseline (Q8_0 q, Q4_0 x Q8_0 dots, online softmax):
    same arguments and result as cpu_baseline_run."""
    n_sess, n_kv, n_ctx, nblk = kc.shape
    d = nblk * 32
    pos = np.ascontiguousarray(pos, dtype=np.int64)
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros((n_sess, n_heads, d), dtype=np.float32)
    secs = lib().orc_cpu_ggml_style_run(_p(kc), _p(vc), n_sess, n_heads, n_kv, d, n_ctx,
                                        _p(pos), _p(q), _p(out), n_threads, iters)
    return float(secs), out
