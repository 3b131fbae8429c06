"""The device generator of the benchmark configurations' inputs
(libbmo_synth.so, include/bmo_synth.h) against the oracle's restatement
(orc_fill_normal / orc_fill_kv): equal bit for bit, with and without the x8
outliers, at offsets near 0 and past 2^40, for the configurations' seeds and
for lengths around the kernel's block and grid sizes."""
import numpy as np
import pytest

import oracle
from bmo_jetson_amd.synth import fill_normal

pytestmark = pytest.mark.gpu

SEEDS = [0xB0A00001, 0xB0A00002, 0xB0A00003, 0xB0A00004, 0xB0A00005, 0, 2**64 - 1]


@pytest.mark.parametrize("seed", SEEDS)
@pytest.mark.parametrize("outliers", [False, True])
def test_synth_matches_oracle(gpu, seed, outliers):
    for n, offset in ((1 << 22, 0), (1 << 20, (1 << 40) + 12345), (257, 7), (1, 2**63)):
        out = gpu.full((n,), float("nan"), dtype=gpu.float32, device="cuda")
        fill_normal(out, seed, offset, outliers)
        gpu.cuda.synchronize()
        got = out.cpu().numpy()
        ref = (oracle.kv_normal if outliers else oracle.normal)(seed, n, offset=offset)
        if not np.array_equal(got.view(np.uint32), ref.view(np.uint32)):
            bad = np.flatnonzero(got.view(np.uint32) != ref.view(np.uint32))
            raise AssertionError(f"seed {seed:#x} offset {offset} n {n}: {bad.size} elements differ, "
                                 f"first {bad[0]}: {got[bad[0]]!r} vs {ref[bad[0]]!r}")


def test_synth_grid_stride(gpu):
    """More elements than one grid pass (65536 blocks x 256 threads)."""
    n = 65536 * 256 + 1000
    out = gpu.empty((n,), dtype=gpu.float32, device="cuda")
    fill_normal(out, 0xB0A00003, 99, True)
    gpu.cuda.synchronize()
    got = out.cpu().numpy()
    tail = oracle.kv_normal(0xB0A00003, 3000, offset=99 + n - 3000)
    assert np.array_equal(got[-3000:].view(np.uint32), tail.view(np.uint32))


def test_read_probe_reads_and_leaves_data(gpu):
    """The bench's read probe (bmo_synth_read_probe) runs over a buffer, on a
    stream, without changing it; its sink is written only when a 16-byte
    piece's xor is 0x9E3779B9, which one planted piece makes happen."""
    from bmo_jetson_amd.synth import read_probe
    n = (1 << 20) + 16                       # not a multiple of the workgroup's 4 KiB
    buf = gpu.zeros(n // 4, dtype=gpu.int32, device="cuda")
    buf[4:8] = gpu.tensor([0x9E3779B9 - (1 << 32), 0, 0, 0], dtype=gpu.int32)  # piece 1
    before = buf.cpu().numpy().copy()
    sink = gpu.zeros(256, dtype=gpu.int32, device="cuda")
    st = gpu.cuda.Stream()
    read_probe(buf.data_ptr(), n, sink, stream=st)
    st.synchronize()
    assert np.array_equal(buf.cpu().numpy(), before)
    got = sink.cpu().numpy()
    assert got[1] == 1 and np.count_nonzero(got) == 1    # piece 1 is read by thread 1
