"""Seeded random shapes for chunked prefill against the float64 oracle (same
bar as tests/test_gpu_prefill.py): head_dim 64 or 128, ring sizes on and off
the 32-slot grid, histories from empty to many wraps, chunks from one token
to the whole ring, and 1, 2 or 4 query heads per kv head.  This reaches the
tile orders (paired ring/chunk tiles, unpaired tails, padding), both
workgroup shapes and both the direct and the staged path."""
import numpy as np
import pytest

from _ringsim import Mirror
from test_gpu_prefill import _run

pytestmark = pytest.mark.gpu

SEEDS = list(range(24))


def _shape(seed):
    r = np.random.default_rng(0xB0A0F000 + seed)
    d = int(r.choice([64, 128]))
    n_ctx = int(r.choice([8, 24, 32, 40, 64, 96, 100, 128, 160, 256]))
    n_kv = int(r.choice([1, 2]))
    n_heads = n_kv * int(r.choice([1, 1, 2, 4]))
    n_tok = int(r.integers(1, min(n_ctx, 128) + 1))
    pos0 = int(r.choice([0, int(r.integers(1, n_ctx)), int(r.integers(n_ctx, 6 * n_ctx))]))
    return d, n_ctx, n_kv, n_heads, n_tok, pos0


@pytest.mark.parametrize("seed", SEEDS)
def test_prefill_random_shape(gpu, seed):
    d, n_ctx, n_kv, n_heads, n_tok, pos0 = _shape(seed)
    m = Mirror(gpu, 1, 1, n_kv, d, n_ctx)
    m.fill_range(0, 0, 0, pos0, seed=500 + seed)
    _run(gpu, m, 0, [(0, pos0)], n_tok, n_heads, seed=600 + seed)
