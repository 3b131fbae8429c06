"""CPU-side checks of the C ABI: the library loads, exports every function
include/bmo_attn.h declares, and the error paths that need no GPU behave as
the reference's ABI does (NULL-safe free, rc 1 for NULL, -1/-2/-3 readout
codes, NULL + message from a rejected create).  No compute is launched."""
import ctypes
import subprocess

import numpy as np
import pytest

import bmo_jetson_amd as bmo
from bmo_jetson_amd import _lib


def test_header_symbols_exported():
    names = bmo.header_symbols()
    assert len(names) >= 17
    L = bmo.lib()
    for n in names:
        assert hasattr(L, n), n
    out = subprocess.run(["nm", "-D", "--defined-only", bmo.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(names) <= exported
    # nothing but the declared ABI is exported from the library's own code
    ours = {s for s in exported if s.startswith("bmo")}
    assert ours == set(names)
    assert set(_lib.SIGNATURES) == set(names)


def test_stripe_bytes():
    L = bmo.lib()
    # K and V of one kv head: groups of 2048/head_dim slots, 2304 bytes each
    # (K codes, V codes, one (K, V) scale dword per block).
    # temporal: 512 slots = 32 groups of 16 = 512 * (64 + 64 + 16) bytes
    assert L.bmo_kv_ring_stripe_bytes(128, 512) == 512 * 144 == 32 * 2304
    # depformer: 8 slots fit one group of 32 (slots 8..31 are padding)
    assert L.bmo_kv_ring_stripe_bytes(64, 8) == 2304
    assert L.bmo_kv_ring_stripe_bytes(128, 17) == 2 * 2304
    assert L.bmo_kv_ring_stripe_bytes(0, 8) == 0
    assert L.bmo_kv_ring_stripe_bytes(96, 8) == 0


@pytest.mark.parametrize("args", [(0, 1, 1, 128, 8), (1, 0, 1, 128, 8), (1, 1, 0, 128, 8),
                                  (1, 1, 1, 96, 8), (1, 1, 1, 128, 0), (1, 1, 1, 128, 65537)])
def test_create_rejects_bad_geometry(args):
    L = bmo.lib()
    assert not L.bmo_kv_ring_create(*args)
    err = L.bmo_kv_ring_last_error(None)
    assert err and err.startswith(b"bmo_kv_ring_create:")


def test_null_handle_paths():
    L = bmo.lib()
    L.bmo_kv_ring_free(None)  # NULL-safe, like bmo_free
    assert L.bmo_kv_ring_geometry(None, None, None, None, None, None) == 1
    assert L.bmo_kv_ring_bytes(None) == 0
    assert L.bmo_kv_ring_k_base(None) is None
    assert L.bmo_kv_ring_reset(None, -1, None) == 1
    assert L.bmo_kv_ring_append(None, 0, 1, None, None, None, None, None) == 1
    assert L.bmo_kv_ring_decode(None, 0, 1, None, None, 1, None, None, 0.0, None) == 1
    assert L.bmo_kv_ring_append_decode(None, 0, 1, None, None, 1, None, None, None, None, 0.0,
                                       None) == 1
    assert L.bmo_kv_ring_append_decode_rope(None, 0, 1, None, None, 1, None, None, None, None,
                                            0.0, 10000.0, None) == 1
    assert L.bmo_kv_ring_write(None, 0, 0, 0, 1, None, None, None) == 1
    assert L.bmo_kv_ring_prefill(None, 0, 1, None, None, 1, 1, None, None, None, None, 0.0,
                                 None) == 1
    buf = np.zeros(16, np.float32)
    assert L.bmo_kv_ring_copy_k_f32(None, 0, 0, 0, 1, buf.ctypes.data, 16) == -1
    assert L.bmo_kv_ring_export_q4_0(None, 0, 0, 0, 0, 1, buf.ctypes.data, 64) == -1
    assert L.bmo_kv_ring_import_q4_0(None, 0, 0, 0, 0, 1, buf.ctypes.data, 64) == -1


def test_node_launcher_rejects_bad_arguments_without_launching():
    # every pointer NULL: returns without touching the device
    bmo.launch_decode_attention(None, None, None, None, None, None, 128, 32, 32, 512, 0, 0)
    # unsupported head_dim with non-NULL (never dereferenced) addresses
    fake = 0x1000
    bmo.launch_decode_attention(fake, fake, fake, fake, fake + 1024, fake, 96, 32, 32, 512, 0, 0)
    # v_cache must be k_cache + 1024 (the V codes' offset inside a slot group)
    bmo.launch_decode_attention(fake, fake, fake, fake, fake + 4096, fake, 128, 32, 32, 512, 0, 0)


def test_package_fails_loudly_without_library(tmp_path, monkeypatch):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.lib()


def test_synth_header_symbols_exported():
    """libbmo_synth.so (the benchmark inputs' generator and read probe)
    exports exactly what include/bmo_synth.h declares, and rejects bad
    arguments without launching."""
    import os
    import re
    from bmo_jetson_amd import synth
    text = open(os.path.join(_lib.ROOT, "include", "bmo_synth.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("#"))
    names = set(re.findall(r"BMO_SYNTH_API\s+[^;(]*?\b(\w+)\s*\(", text))
    assert names == {"bmo_synth_fill_normal", "bmo_synth_read_probe"}
    out = subprocess.run(["nm", "-D", "--defined-only", synth.SYNTH_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert {s for s in exported if s.startswith("bmo")} == names
    L = synth.lib()
    assert L.bmo_synth_fill_normal(None, -1, 0, 0, 0, None) == 2
    assert L.bmo_synth_fill_normal(None, 5, 0, 0, 0, None) == 2
    assert L.bmo_synth_fill_normal(None, 0, 0, 0, 0, None) == 0
    assert L.bmo_synth_read_probe(None, -16, None, None) == 2
    assert L.bmo_synth_read_probe(None, 16, None, None) == 2           # NULL buffer
    assert L.bmo_synth_read_probe(ctypes.c_void_p(16), 24, ctypes.c_void_p(16), None) == 2  # not whole pieces
    assert L.bmo_synth_read_probe(ctypes.c_void_p(8), 16, ctypes.c_void_p(16), None) == 2   # misaligned
    assert L.bmo_synth_read_probe(None, 0, None, None) == 0
