"""Python view of the Q4_0 ring (ctypes over include/bmo_attn.h).

Mirrors the KV-touching part of the reference's Python binding
(``bmo_engine.py``): ``reset`` (bmo_engine.py:135-137) and
``get_k_cache_f32`` (bmo_engine.py:258-280, same layout
``(n_positions, n_heads, head_dim)`` and the same errors), plus the batched
append / decode entry points that the reference's single-session handle does
not have.
"""
from __future__ import annotations

import ctypes

import numpy as np

from ._lib import lib

BLOCK_Q4_0_BYTES = 18


class RingError(RuntimeError):
    def __init__(self, fn: str, rc: int, msg: str | None):
        super().__init__(f"{fn} rc={rc}: {msg or 'unknown'}")
        self.rc = rc
        self.msg = msg or ""


def _ptr(x) -> int | None:
    """Device (or host) address of a tensor / int / None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return int(x.data_ptr())
    raise TypeError(f"expected a tensor, an int address or None, got {type(x)!r}")


def _stream(s) -> int | None:
    if s is None:
        return None
    if isinstance(s, int):
        return s
    if hasattr(s, "cuda_stream"):
        return int(s.cuda_stream)
    raise TypeError(f"expected a stream, an int handle or None, got {type(s)!r}")


def stripe_bytes(head_dim: int, n_ctx: int) -> int:
    return int(lib().bmo_kv_ring_stripe_bytes(head_dim, n_ctx))


class KVRing:
    """A device-resident Q4_0 ring: [n_layers][n_sessions][n_kv_heads] stripes
    of n_ctx slots.  The reference's temporal cache is
    ``KVRing(32, 1, 32, 128, 512)``, its depformer cache ``KVRing(6, 1, 16, 64, 8)``.
    """

    def __init__(self, n_layers: int, n_sessions: int, n_kv_heads: int, head_dim: int,
                 n_ctx: int):
        L = lib()
        h = L.bmo_kv_ring_create(n_layers, n_sessions, n_kv_heads, head_dim, n_ctx)
        if not h:
            err = L.bmo_kv_ring_last_error(None)
            raise RuntimeError(f"bmo_kv_ring_create failed: {err.decode() if err else 'unknown'}")
        self._h = h
        # bound here so that __del__ never needs module globals, which the
        # interpreter may already have cleared when it runs at exit
        self._free = L.bmo_kv_ring_free
        self.n_layers = n_layers
        self.n_sessions = n_sessions
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.n_ctx = n_ctx

    # -- lifetime ---------------------------------------------------------------
    def close(self) -> None:
        h = getattr(self, "_h", None)
        if h:
            self._h = None
            self._free(h)

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter teardown: nothing left to report to
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def handle(self) -> int:
        return self._h

    @property
    def nbytes(self) -> int:
        return int(lib().bmo_kv_ring_bytes(self._h))

    @property
    def k_base(self) -> int:
        return int(lib().bmo_kv_ring_k_base(self._h))

    @property
    def v_base(self) -> int:
        return int(lib().bmo_kv_ring_v_base(self._h))

    def geometry(self):
        vals = [ctypes.c_int() for _ in range(5)]
        rc = lib().bmo_kv_ring_geometry(self._h, *[ctypes.byref(v) for v in vals])
        self._check("bmo_kv_ring_geometry", rc)
        return tuple(v.value for v in vals)

    def last_error(self) -> str | None:
        e = lib().bmo_kv_ring_last_error(self._h)
        return e.decode() if e else None

    def _check(self, fn: str, rc: int) -> None:
        if rc != 0:
            raise RingError(fn, rc, self.last_error())

    # -- state ------------------------------------------------------------------
    def reset(self, session: int = -1, stream=None) -> None:
        self._check("bmo_kv_ring_reset",
                    lib().bmo_kv_ring_reset(self._h, session, _stream(stream)))

    # -- decode path ------------------------------------------------------------
    def append(self, layer: int, pos, k, v, session_ids=None, n_batch=None, stream=None):
        n = self._batch(pos, n_batch)
        self._check("bmo_kv_ring_append", lib().bmo_kv_ring_append(
            self._h, layer, n, _ptr(session_ids), _ptr(pos), _ptr(k), _ptr(v), _stream(stream)))

    def decode(self, layer: int, pos, q, out, n_heads: int, session_ids=None, scale: float = 0.0,
               n_batch=None, stream=None):
        n = self._batch(pos, n_batch)
        self._check("bmo_kv_ring_decode", lib().bmo_kv_ring_decode(
            self._h, layer, n, _ptr(session_ids), _ptr(pos), n_heads, _ptr(q), _ptr(out),
            float(scale), _stream(stream)))

    def append_decode(self, layer: int, pos, q, k, v, out, n_heads: int, session_ids=None,
                      scale: float = 0.0, n_batch=None, stream=None, rope_theta: float | None = None):
        """Fused append + attention.  With rope_theta, q and k are the pre-RoPE
        rows and interleaved RoPE at each entry's position is applied first
        (bmo_kv_ring_append_decode_rope)."""
        n = self._batch(pos, n_batch)
        if rope_theta is None:
            self._check("bmo_kv_ring_append_decode", lib().bmo_kv_ring_append_decode(
                self._h, layer, n, _ptr(session_ids), _ptr(pos), n_heads, _ptr(q), _ptr(k), _ptr(v),
                _ptr(out), float(scale), _stream(stream)))
        else:
            self._check("bmo_kv_ring_append_decode_rope", lib().bmo_kv_ring_append_decode_rope(
                self._h, layer, n, _ptr(session_ids), _ptr(pos), n_heads, _ptr(q), _ptr(k), _ptr(v),
                _ptr(out), float(scale), float(rope_theta), _stream(stream)))

    def write(self, layer: int, session: int, pos0: int, k, v, n_tok=None, stream=None):
        if n_tok is None:
            n_tok = int(k.shape[0])
        self._check("bmo_kv_ring_write", lib().bmo_kv_ring_write(
            self._h, layer, session, int(pos0), int(n_tok), _ptr(k), _ptr(v), _stream(stream)))

    def prefill(self, layer: int, pos0, q, k, v, out, n_heads: int, n_tok: int | None = None,
                session_ids=None, scale: float = 0.0, n_batch=None, stream=None):
        """Chunked prefill: q [n_batch][n_tok][n_heads][d], k/v
        [n_batch][n_tok][n_kv][d] as bf16 tensors (or raw bf16 addresses),
        out [n_batch][n_tok][n_heads][d] fp32; pos0 a device int32 [n_batch]."""
        n = self._batch(pos0, n_batch)
        if n_tok is None:
            n_tok = int(q.shape[-3]) if hasattr(q, "shape") and q.dim() >= 3 else None
            if n_tok is None:
                raise ValueError("n_tok is required when q is a raw address")
        self._check("bmo_kv_ring_prefill", lib().bmo_kv_ring_prefill(
            self._h, layer, n, _ptr(session_ids), _ptr(pos0), int(n_tok), n_heads, _ptr(q),
            _ptr(k), _ptr(v), _ptr(out), float(scale), _stream(stream)))

    @staticmethod
    def _batch(pos, n_batch):
        if n_batch is not None:
            return int(n_batch)
        if hasattr(pos, "numel"):
            return int(pos.numel())
        raise ValueError("n_batch is required when pos is a raw address")

    # -- readout ------------------------------------------------------------------
    def copy_k_cache_f32(self, layer: int, t_start: int, n_positions: int, out: np.ndarray,
                         session: int = 0) -> int:
        """The raw call (bmo_copy_k_cache_f32 contract): returns the count or a
        negative code."""
        assert out.dtype == np.float32 and out.flags["C_CONTIGUOUS"]
        return int(lib().bmo_kv_ring_copy_k_f32(self._h, layer, session, t_start, n_positions,
                                                out.ctypes.data, int(out.size)))

    def get_k_cache_f32(self, layer: int, t_start: int, n_positions: int,
                        session: int = 0) -> np.ndarray:
        """K slots as float32, layout (n_positions, n_kv_heads, head_dim)
        (bmo_engine.py:258-280)."""
        n_el = int(n_positions) * self.n_kv_heads * self.head_dim
        buf = np.empty(max(n_el, 1), dtype=np.float32)
        n_written = self.copy_k_cache_f32(layer, t_start, n_positions, buf, session)
        if n_written < 0:
            raise RuntimeError(f"bmo_copy_k_cache_f32 failed with code {n_written}")
        if n_written != n_el:
            raise RuntimeError(f"bmo_copy_k_cache_f32 expected {n_el} floats, got {n_written}")
        return buf[:n_el].reshape(int(n_positions), self.n_kv_heads, self.head_dim)

    def export_q4_0(self, layer: int, session: int, which: int, t_start: int,
                    n_positions: int) -> np.ndarray:
        """ggml block_q4_0 bytes, shape (n_positions, n_kv_heads, head_dim/32, 18)."""
        nblk = self.head_dim // 32
        shape = (n_positions, self.n_kv_heads, nblk, BLOCK_Q4_0_BYTES)
        buf = np.zeros(shape, dtype=np.uint8)
        rc = lib().bmo_kv_ring_export_q4_0(self._h, layer, session, which, t_start, n_positions,
                                           buf.ctypes.data, buf.size)
        if rc < 0:
            raise RuntimeError(f"bmo_kv_ring_export_q4_0 failed with code {rc}")
        return buf

    def import_q4_0(self, layer: int, session: int, which: int, t_start: int,
                    blocks: np.ndarray) -> None:
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        nblk = self.head_dim // 32
        n_positions = blocks.size // (self.n_kv_heads * nblk * BLOCK_Q4_0_BYTES)
        rc = lib().bmo_kv_ring_import_q4_0(self._h, layer, session, which, t_start, n_positions,
                                           blocks.ctypes.data, blocks.size)
        if rc < 0:
            raise RuntimeError(f"bmo_kv_ring_import_q4_0 failed with code {rc}")


class Session:
    """Per-session handle (bmo_attn_session_*): one session of a ring with its
    own HIP stream and device position; ``forward`` runs one token's fused
    append + attention through every layer at a position and advances it,
    ``capture`` / ``replay`` do the same from a HIP graph recorded in the
    library.  q/out are [n_layers][n_heads][head_dim] and k/v
    [n_layers][n_kv_heads][head_dim] fp32 device buffers.

    At a model's layer granularity, ``begin_step(pos)``, ``layer(l, q, k, v,
    out)`` per layer and ``end_step()`` queue the step one layer at a time on
    ``stream``, where the caller's own kernels (projections, FFN) fall
    between them; ``capture_begin()`` / ``capture_end()`` record whatever is
    queued on the stream in between (a frame may start with
    ``reset_async()``), and ``replay`` runs it."""

    def __init__(self, ring: KVRing, session: int, n_heads: int, scale: float = 0.0,
                 rope_theta: float = 0.0):
        L = lib()
        h = L.bmo_attn_session_create(ring.handle, session, n_heads, float(scale),
                                      float(rope_theta))
        if not h:
            err = L.bmo_attn_session_last_error(None)
            raise RuntimeError(f"bmo_attn_session_create failed: {err.decode() if err else 'unknown'}")
        self._h = h
        self._free = L.bmo_attn_session_free
        self.ring = ring  # the ring must outlive the handle
        self.session = session
        self.n_heads = n_heads

    def close(self) -> None:
        h = getattr(self, "_h", None)
        if h:
            self._h = None
            self._free(h)

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter teardown
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def handle(self) -> int:
        return self._h

    def last_error(self) -> str | None:
        e = lib().bmo_attn_session_last_error(self._h)
        return e.decode() if e else None

    def _check(self, fn: str, rc: int) -> None:
        if rc != 0:
            raise RingError(fn, rc, self.last_error())

    @property
    def pos(self) -> int:
        return int(lib().bmo_attn_session_pos(self._h))

    @property
    def stream(self) -> int:
        return int(lib().bmo_attn_session_stream(self._h) or 0)

    def reset(self) -> None:
        self._check("bmo_attn_session_reset", lib().bmo_attn_session_reset(self._h))

    def forward(self, pos: int, q, k, v, out) -> None:
        self._check("bmo_attn_session_forward", lib().bmo_attn_session_forward(
            self._h, int(pos), _ptr(q), _ptr(k), _ptr(v), _ptr(out)))

    def capture(self, q, k, v, out) -> None:
        self._check("bmo_attn_session_capture", lib().bmo_attn_session_capture(
            self._h, _ptr(q), _ptr(k), _ptr(v), _ptr(out)))

    @property
    def has_graph(self) -> bool:
        return bool(lib().bmo_attn_session_has_graph(self._h))

    def replay(self, pos: int = 0) -> None:
        self._check("bmo_attn_session_replay", lib().bmo_attn_session_replay(self._h, int(pos)))

    def begin_step(self, pos: int) -> None:
        self._check("bmo_attn_session_begin_step", lib().bmo_attn_session_begin_step(self._h, int(pos)))

    def layer(self, layer: int, q, k, v, out) -> None:
        self._check("bmo_attn_session_layer", lib().bmo_attn_session_layer(
            self._h, int(layer), _ptr(q), _ptr(k), _ptr(v), _ptr(out)))

    def end_step(self) -> None:
        self._check("bmo_attn_session_end_step", lib().bmo_attn_session_end_step(self._h))

    def reset_async(self) -> None:
        self._check("bmo_attn_session_reset_async", lib().bmo_attn_session_reset_async(self._h))

    def sync(self) -> None:
        self._check("bmo_attn_session_sync", lib().bmo_attn_session_sync(self._h))

    def capture_begin(self) -> None:
        self._check("bmo_attn_session_capture_begin", lib().bmo_attn_session_capture_begin(self._h))

    def capture_end(self) -> None:
        self._check("bmo_attn_session_capture_end", lib().bmo_attn_session_capture_end(self._h))


def launch_decode_attention(q, k, v, k_cache, v_cache, out, head_dim: int, n_heads: int,
                            n_kv_heads: int, n_ctx: int, n_past: int, layer: int, stream=None,
                            pos_dev=None) -> None:
    """The node-level drop-in (reference launch_decode_attention signature)."""
    lib().bmo_launch_decode_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache),
                                      _ptr(out), head_dim, n_heads, n_kv_heads, n_ctx, n_past,
                                      layer, _stream(stream), _ptr(pos_dev))


def positions_advance(pos, n: int, delta: int = 1, stream=None) -> None:
    """pos[i] += delta on the device (capturable: a graph of a decode step
    ending with it advances its own positions on every replay)."""
    rc = lib().bmo_positions_advance(_ptr(pos), int(n), int(delta), _stream(stream))
    if rc != 0:
        raise RingError("bmo_positions_advance", rc, None)


def gemv_q4_0_q8_1(w, x, y, rows: int, cols: int, q8_scratch=None, stream=None) -> None:
    """y = W x for ggml Q4_0 weights W (rows x cols, device bytes) and fp32 x,
    with x quantized to the reference's Q8_1 (bmo_launch_gemv_q4_0_q8_1)."""
    rc = lib().bmo_launch_gemv_q4_0_q8_1(_ptr(w), _ptr(x), _ptr(y), int(rows), int(cols),
                                         _ptr(q8_scratch), _stream(stream))
    if rc != 0:
        raise RingError("bmo_launch_gemv_q4_0_q8_1", rc, None)
